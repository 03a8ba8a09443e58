"""The oracle and the package's CPU fallbacks against golden vectors written
by the reference's own CPU fallbacks (tests/golden/make_golden.py: seeded
inputs through trishitmg/neural_shift_cuda ops.py / metropolis.py).

What each check pins:

* accumulate_uz, accumulate_uz_scalar (fp16/fp32/fp64): the oracle and the
  package fallback reproduce the reference fallback's U and Z bit for bit,
  so the term order [fwd_0, inv_0?, ...] and the pairwise tree
  (ops.py:77-92, 157-206, 350-390) are pinned exactly; gradients agree with
  the reference's autograd within the accumulation tolerance (the oracle's
  analytic adjoint, shift_ops_cuda.cu:343-458, sums in another order).
* gathers (fp32/fp64/fp16/bf16, R = 0 branch): bit-exact outputs and masks,
  mask dtype equal to the guide dtype (ops.py:95-154); backward within the
  tolerance of a dtype-precision sum.
* normalized_accumulate_uz: D and log_C within tolerance (exp/log come from
  different libraries), NaN / -inf patterns exactly: empty rows give D = 0,
  log_C = -inf; out-of-contract weights with validate=False follow the
  reference CPU rule.  The reference fallback's NaN weight gradient at an
  exact-zero positive weight (ops.py:227-231) is pinned as such; the package
  returns 0 there (the reference GPU kernel's rule, shift_ops_cuda.cu:748-751).
* metropolis_aggregate: Wx and d_hat of the reference dispatcher and of its
  torch restatement; gradients of the checkpointed training path.
"""
from __future__ import annotations

import pytest
import torch

import oracle
from helpers import (assert_bound, golden_cases, golden_names, metropolis_grad_abs,
                     normalized_bwd_cond, out_ulp_for, rtol_for)
from neural_shift_cuda import (accumulate_uz, accumulate_uz_scalar, metropolis_aggregate,
                               normalized_accumulate_uz, pair_gather, shift_gather)


def _acc(dtype):
    return torch.float64 if dtype == torch.float64 else torch.float32


def test_golden_fixture_inventory():
    ops = {}
    for c in golden_cases().values():
        ops[c["op"]] = ops.get(c["op"], 0) + 1
    assert ops == {"accumulate_uz": 5, "normalized_accumulate_uz": 6, "shift_gather": 3,
                   "pair_gather": 3, "accumulate_uz_scalar": 2, "metropolis_aggregate": 5,
                   "accumulate_uz_config": 1, "nectr_installer": 2, "nekde_installer": 13,
                   "gasd_installer": 6, "metropolis_installer": 2}


# ---------------------------------------------------------------------------
# accumulate_uz
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name", golden_names("accumulate_uz"))
def test_oracle_accumulate_bit_exact(name):
    c = golden_cases()[name]
    I, O = c["inputs"], c["outputs"]
    acc = _acc(I["x"].dtype)
    U, Z = oracle.accumulate_uz(I["x"], I["w"], I["shifts"], dtype=acc)
    assert U.dtype == O["U"].dtype == acc
    assert torch.equal(U, O["U"]), f"{name}: U differs from the reference bits"
    assert torch.equal(Z, O["Z"]), f"{name}: Z differs from the reference bits"


@pytest.mark.parametrize("name", golden_names("accumulate_uz"))
def test_oracle_accumulate_grads(name):
    c = golden_cases()[name]
    I, O = c["inputs"], c["outputs"]
    x, w, sh = I["x"], I["w"], I["shifts"]
    gx, gw = oracle.accumulate_uz_bwd(x, w, I["gU"], I["gZ"], sh)
    gxs, gws = oracle.accumulate_uz_bwd(x.abs(), w.abs(), I["gU"].abs(), I["gZ"].abs(), sh)
    rt = rtol_for(x.dtype)
    assert O["gx"].dtype == x.dtype and O["gw"].dtype == w.dtype
    assert_bound(O["gx"], gx, gxs, rt, f"{name} gx", out_ulp_for(x.dtype))
    assert_bound(O["gw"], gw, gws, rt, f"{name} gw", out_ulp_for(w.dtype))


@pytest.mark.parametrize("name", golden_names("accumulate_uz"))
def test_fallback_accumulate(name):
    c = golden_cases()[name]
    I, O = c["inputs"], c["outputs"]
    xr = I["x"].clone().requires_grad_(True)
    wr = I["w"].clone().requires_grad_(True)
    U, Z = accumulate_uz(xr, wr, I["shifts"])
    assert torch.equal(U.detach(), O["U"]) and torch.equal(Z.detach(), O["Z"])
    torch.autograd.backward([U, Z], [I["gU"], I["gZ"]])
    gxs, gws = oracle.accumulate_uz_bwd(I["x"].abs(), I["w"].abs(), I["gU"].abs(),
                                        I["gZ"].abs(), I["shifts"])
    rt = rtol_for(I["x"].dtype)
    ou = out_ulp_for(I["x"].dtype)
    assert_bound(xr.grad, O["gx"], gxs, rt, f"{name} gx", ou)
    assert_bound(wr.grad, O["gw"], gws, rt, f"{name} gw", ou)


# ---------------------------------------------------------------------------
# accumulate_uz_scalar
# ---------------------------------------------------------------------------

def _scalar_w3(I):
    w = I["w"]
    if w.dim() == 2:
        w = w.unsqueeze(-1).expand(w.shape[0], w.shape[1], I["x"].shape[1])
    return w.contiguous()


@pytest.mark.parametrize("name", golden_names("accumulate_uz_scalar"))
def test_oracle_scalar(name):
    c = golden_cases()[name]
    I, O = c["inputs"], c["outputs"]
    w3 = _scalar_w3(I)
    U, Z = oracle.accumulate_uz_scalar(I["x"], w3, I["shifts"], dtype=_acc(I["x"].dtype))
    assert torch.equal(U, O["U"]) and torch.equal(Z, O["Z"])
    gx, gw3 = oracle.accumulate_uz_scalar_bwd(I["x"], w3, I["gU"], I["gZ"], I["shifts"])
    gxs, gws3 = oracle.accumulate_uz_scalar_bwd(I["x"].abs(), w3.abs(), I["gU"].abs(),
                                                I["gZ"].abs(), I["shifts"])
    if I["w"].dim() == 2:  # (S, B) weights: the gradient sums over channels
        gw3, gws3 = gw3.sum(-1), gws3.sum(-1)
    rt = rtol_for(I["x"].dtype)
    assert_bound(O["gx"], gx, gxs, rt, f"{name} gx")
    assert_bound(O["gw"], gw3, gws3, rt, f"{name} gw")


@pytest.mark.parametrize("name", golden_names("accumulate_uz_scalar"))
def test_fallback_scalar(name):
    c = golden_cases()[name]
    I, O = c["inputs"], c["outputs"]
    U, Z = accumulate_uz_scalar(I["x"], I["w"], I["shifts"])
    assert torch.equal(U, O["U"]) and torch.equal(Z, O["Z"])


# ---------------------------------------------------------------------------
# gathers
# ---------------------------------------------------------------------------

_GATHER_NAMES = golden_names("shift_gather") + golden_names("pair_gather")


@pytest.mark.parametrize("name", _GATHER_NAMES)
def test_oracle_gathers_bit_exact(name):
    c = golden_cases()[name]
    I, O = c["inputs"], c["outputs"]
    fn = oracle.shift_gather if c["op"] == "shift_gather" else oracle.pair_gather
    out, mask = fn(I["guide"], I["shifts"])
    assert out.dtype == mask.dtype == I["guide"].dtype == O["mask"].dtype
    assert torch.equal(out, O["out"]) and torch.equal(mask, O["mask"])


def _gather_grad_check(name, got):
    c = golden_cases()[name]
    I, O = c["inputs"], c["outputs"]
    B, C, H, W = I["guide"].shape
    bwd = oracle.shift_gather_bwd if c["op"] == "shift_gather" else oracle.pair_gather_bwd
    exp = bwd(I["gout"], I["shifts"], B, C, H, W)
    scale = bwd(I["gout"].abs(), I["shifts"], B, C, H, W)
    dt = I["guide"].dtype
    # the reference's autograd sums in the guide dtype: up to S roundings
    terms = I["shifts"].size(0) + 1
    rt = {torch.bfloat16: terms * 2.0 ** -8, torch.float16: terms * 2.0 ** -11}.get(
        dt, rtol_for(dt))
    assert_bound(got, exp, scale, rt, f"{name} grad")


@pytest.mark.parametrize("name", _GATHER_NAMES)
def test_golden_gather_grads_vs_oracle(name):
    _gather_grad_check(name, golden_cases()[name]["outputs"]["gguide"])


@pytest.mark.parametrize("name", _GATHER_NAMES)
def test_fallback_gathers(name):
    c = golden_cases()[name]
    I, O = c["inputs"], c["outputs"]
    fn = shift_gather if c["op"] == "shift_gather" else pair_gather
    g = I["guide"].clone().requires_grad_(True)
    out, mask = fn(g, I["shifts"])
    assert torch.equal(out.detach(), O["out"]) and torch.equal(mask, O["mask"])
    out.backward(I["gout"])
    _gather_grad_check(name, g.grad)


# ---------------------------------------------------------------------------
# normalized_accumulate_uz
# ---------------------------------------------------------------------------

def _normalized_scale(I, log_weights):
    Ds, _ = oracle.normalized(I["x"].abs(), I["w"], I["shifts"], log_weights=log_weights,
                              policy="cpu")
    return Ds


@pytest.mark.parametrize("name", golden_names("normalized_accumulate_uz"))
def test_oracle_normalized_forward(name):
    c = golden_cases()[name]
    I, O = c["inputs"], c["outputs"]
    lw = c["log_weights"]
    D, L = oracle.normalized(I["x"], I["w"], I["shifts"], log_weights=lw, policy="cpu")
    rt = rtol_for(I["x"].dtype)
    assert_bound(O["D"], D, _normalized_scale(I, lw).nan_to_num(), rt, f"{name} D")
    if "log_C" in O:
        assert_bound(O["log_C"], L, L.abs().nan_to_num(posinf=0, neginf=0) + 1.0, rt,
                     f"{name} log_C")


def test_golden_empty_rows_policy():
    """Empty rows: D = 0, log_C = -inf, zero weight gradient; the reference
    fallback's x gradient there is 0/0 = NaN (the GPU kernels give 0)."""
    c = golden_cases()["nrm_log_f64_empty_rows"]
    D, L = c["outputs"]["D"], c["outputs"]["log_C"]
    assert torch.equal(D[1], torch.zeros_like(D[1]))
    assert bool(torch.isneginf(L[1]).all()) and bool(torch.isfinite(L[0]).all())
    gw = c["outputs"]["gw"].view(-1, 2, *D.shape[1:])
    assert torch.equal(gw[:, 1], torch.zeros_like(gw[:, 1]))
    assert bool(torch.isnan(c["outputs"]["gx"][1]).all())
    assert not bool(torch.isnan(c["outputs"]["gx"][0]).any())


def _cuda_rule_grads(I, O, lw, L):
    """The golden gradients with the reference fallback's two NaN quirks
    (zero positive weight -> NaN weight gradient; empty row -> NaN x
    gradient) replaced by the GPU kernels' 0, after checking that the NaNs
    sit exactly there."""
    gx, gw = O["gx"], O["gw"]
    empty = torch.isneginf(L)
    assert torch.equal(torch.isnan(gx), empty)
    gx = torch.where(empty, torch.zeros_like(gx), gx)
    if not lw:
        zero = I["w"] == 0
        assert torch.equal(torch.isnan(gw), zero)
        gw = torch.where(zero, torch.zeros_like(gw), gw)
    else:
        assert not bool(torch.isnan(gw).any())
    return gx, gw


def test_golden_huge_uniform_weights_is_mean():
    c = golden_cases()["nrm_pos_f64_window_huge"]
    x = c["inputs"]["x"]
    mean = sum(torch.roll(x, (-dx, -dy), (-2, -1)) for dx in (-1, 0, 1) for dy in (-1, 0, 1)) / 9
    torch.testing.assert_close(c["outputs"]["D"], mean, rtol=1e-12, atol=1e-12)


def test_golden_zero_weight_gradient_quirk():
    """Reference fallback: NaN gradient exactly where a positive weight is 0."""
    c = golden_cases()["nrm_pos_f64_half_r2"]
    gw, w = c["outputs"]["gw"], c["inputs"]["w"]
    assert int((w == 0).sum()) > 0
    assert torch.equal(torch.isnan(gw), w == 0)


@pytest.mark.parametrize("name", [n for n in golden_names("normalized_accumulate_uz")
                                  if "gw" in golden_cases()[n]["outputs"]])
def test_oracle_normalized_grads(name):
    c = golden_cases()[name]
    I, O = c["inputs"], c["outputs"]
    lw = c["log_weights"]
    x, w, sh = I["x"], I["w"], I["shifts"]
    D, L = oracle.normalized(x, w, sh, log_weights=lw, policy="cpu")
    gL = I.get("gL", torch.zeros_like(I["gD"]))
    gx, gw = oracle.normalized_bwd(x, w, D, L, I["gD"], gL, sh, log_weights=lw)
    Ds = _normalized_scale(I, lw)
    gxs, gws = oracle.normalized_bwd(x.abs(), w, -Ds, L, I["gD"].abs(), gL.abs(), sh,
                                     log_weights=lw)
    rt = rtol_for(x.dtype)
    gx_ref, gw_ref = _cuda_rule_grads(I, O, lw, L)
    # the golden gradients were computed in the accumulator precision through
    # exp(key - max) and the log of their own sums: their fractions carry the
    # derived conditioning term (the oracle's fp64 ones do not)
    gxc, gwc = normalized_bwd_cond(x, w, L, I["gD"], gL, Ds, sh, log_weights=lw,
                                   acc_dtype=x.dtype)
    assert_bound(gx_ref, gx, gxs, rt, f"{name} gx", extra=gxc)
    assert_bound(gw_ref, gw, gws, rt, f"{name} gw", extra=gwc)


@pytest.mark.parametrize("name", golden_names("normalized_accumulate_uz"))
def test_fallback_normalized(name):
    c = golden_cases()[name]
    I, O = c["inputs"], c["outputs"]
    lw = c["log_weights"]
    grads = "gw" in O
    xr = I["x"].clone().requires_grad_(grads)
    wr = I["w"].clone().requires_grad_(grads)
    out = normalized_accumulate_uz(xr, wr, I["shifts"], log_weights=lw,
                                   return_log_degree=c["return_log_degree"],
                                   validate=c["validate"])
    D = out[0] if c["return_log_degree"] else out
    # same term order and library exp/log as the reference: bit-exact
    assert torch.equal(D.detach().nan_to_num(), O["D"].nan_to_num())
    assert torch.equal(torch.isnan(D.detach()), torch.isnan(O["D"]))
    if c["return_log_degree"]:
        L = out[1].detach()
        assert torch.equal(L.nan_to_num(), O["log_C"].nan_to_num())
        assert torch.equal(torch.isnan(L), torch.isnan(O["log_C"]))
    if not grads:
        return
    if c["return_log_degree"]:
        torch.autograd.backward([out[0], out[1]], [I["gD"], I["gL"]])
    else:
        out.backward(I["gD"])
    rt = rtol_for(I["x"].dtype)
    Ds = _normalized_scale(I, lw)
    D64, L64 = oracle.normalized(I["x"], I["w"], I["shifts"], log_weights=lw, policy="cpu")
    gL = I.get("gL", torch.zeros_like(I["gD"]))
    gxs, gws = oracle.normalized_bwd(I["x"].abs(), I["w"], -Ds, L64, I["gD"].abs(), gL.abs(),
                                     I["shifts"], log_weights=lw)
    gx_ref, gw_ref = _cuda_rule_grads(I, O, lw, L64)
    # both sides evaluate their fractions in the accumulator precision: twice
    # the derived conditioning term and twice rtol
    gxc, gwc = normalized_bwd_cond(I["x"], I["w"], L64, I["gD"], gL, Ds, I["shifts"],
                                   log_weights=lw, acc_dtype=I["x"].dtype)
    assert_bound(xr.grad, gx_ref, gxs, 2 * rt, f"{name} gx", extra=2 * gxc)
    assert_bound(wr.grad, gw_ref, gws, 2 * rt, f"{name} gw", extra=2 * gwc)


# ---------------------------------------------------------------------------
# metropolis_aggregate
# ---------------------------------------------------------------------------

def _metro_scale(I, use_box, d_hat):
    Ws, _ = oracle.metropolis(I["w_half"], I["img"].abs(), I["shifts"], use_box)
    return Ws.abs() + 2 * I["img"].double().abs() * (1 + d_hat.double().abs())


@pytest.mark.parametrize("name", golden_names("metropolis_aggregate"))
def test_oracle_metropolis(name):
    c = golden_cases()[name]
    I, O = c["inputs"], c["outputs"]
    ub = c["use_box"]
    Wx, dh = oracle.metropolis(I["w_half"], I["img"], I["shifts"], ub, eps=c["eps"])
    rt = rtol_for(I["img"].dtype)
    scale = _metro_scale(I, ub, dh)
    for key_wx, key_dh in (("Wx", "d_hat"), ("Wx_torch", "d_hat_torch"),
                           ("Wx_train", "d_hat_train")):
        assert_bound(O[key_wx], Wx, scale, rt, f"{name} {key_wx}")
        assert_bound(O[key_dh], dh, dh.abs(), rt, f"{name} {key_dh}")


@pytest.mark.parametrize("name", golden_names("metropolis_aggregate"))
def test_fallback_metropolis(name):
    c = golden_cases()[name]
    I, O = c["inputs"], c["outputs"]
    ub = c["use_box"]
    rows = [(dx, dy, bool(inv)) for dx, dy, inv in I["shifts"].tolist()]
    with torch.no_grad():
        Wx, dh = metropolis_aggregate(I["w_half"], I["img"], rows, ub)
    rt = rtol_for(I["img"].dtype)
    scale = _metro_scale(I, ub, O["d_hat"])
    assert_bound(Wx, O["Wx"], scale, rt, f"{name} Wx")
    assert_bound(dh, O["d_hat"], O["d_hat"].abs(), rt, f"{name} d_hat")
    wr = I["w_half"].clone().requires_grad_(True)
    ir = I["img"].clone().requires_grad_(True)
    Wg, dg = metropolis_aggregate(wr, ir, rows, ub, checkpoint_train=True)
    torch.autograd.backward([Wg, dg], [I["gWx"], I["gDh"]])
    # per-element scale: the gradient expressions on absolute values; both
    # sides ran the same graph in the same precision: twice the bound
    gscale_w, gscale_i = metropolis_grad_abs(I["w_half"], I["img"], I["gWx"], I["gDh"],
                                             rows, ub, c["eps"])
    assert_bound(wr.grad, O["g_w_half"], gscale_w, rt * 2, f"{name} g_w_half")
    assert_bound(ir.grad, O["g_img"], gscale_i, rt * 2, f"{name} g_img")


# ---------------------------------------------------------------------------
# BASELINE configs[0] at full size (fp32 1x1x256^2, R=3 half-plane, comp_box):
# the reference dispatcher's CPU forward, regenerated inputs tied to the
# stored outputs by their digest
# ---------------------------------------------------------------------------

def c0_golden():
    from neural_shift_cuda_amd.workloads import config0_inputs, tensor_digest
    c = golden_cases()["c0_full"]
    x, w, sh = config0_inputs()
    assert tensor_digest(x, w, sh) == c["inputs_sha256"], "c0 inputs differ from the digest"
    assert torch.equal(sh, c["inputs"]["shifts"])
    return x, w, sh, c["outputs"]


def test_c0_full_size_bit_exact():
    x, w, sh, O = c0_golden()
    U, Z = oracle.accumulate_uz(x, w, sh, dtype=torch.float32)
    assert torch.equal(U, O["U"]) and torch.equal(Z, O["Z"]), "oracle differs from the reference"
    U, Z = accumulate_uz(x, w, sh)  # the package's CPU fallback
    assert U.dtype == torch.float32
    assert torch.equal(U, O["U"]) and torch.equal(Z, O["Z"]), "fallback differs from the reference"
