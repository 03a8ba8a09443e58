"""BASELINE.json configurations c0-c4 at their full sizes on the GPU, checked
against the CPU oracle.

* c0: accumulate_uz, fp32 1x1x256^2, R=3 half-plane (S=25), comp_box,
  softplus weights: the HIP forward against the reference's own CPU output
  at full size (golden vectors) and the oracle, plus the backward.

* c1: shift_gather + pair_gather, bf16, B=8 C=3 256^2, R=5: box mode (61
  half-plane rows, mask used) and periodic mode (121 window rows); bit-exact,
  backward within tolerance.
* c2: fp16 (fp32 accumulation), B=4 C=1 512^2, R=7 (S=113): accumulate_uz and
  normalized_accumulate_uz (log weights N(0, var 4) with 1% set to +-80)
  fwd+bwd with N(0,1) upstream gradients, against the full-size oracle.
* c3: GASD full window (121 rows), fp32 B=16 C=3 256^2, softplus weights,
  comp_box on and off: U/Z and D = U/Z fwd+bwd; plus fp64 at B=2 at 1e-12.
* c4: 8192^2, S=85, fp32: accumulate_uz fwd+bwd (S*B*C*H*W = 5.7e9 > 2^31,
  the int64 stress) and metropolis_aggregate, checked on random 256x256
  crops with the window oracle (global wrap and box rules); Metropolis W is
  checked for exact symmetry with basis vectors.
"""
from __future__ import annotations

import sys

import pytest
import torch

import oracle
from helpers import assert_bound, normalized_bwd_cond, out_ulp_for, rtol_for
from neural_shift_cuda import (accumulate_uz, metropolis_aggregate, normalized_accumulate_uz,
                               pair_gather, shift_gather)
from neural_shift_cuda_amd.workloads import (box_stack, halfplane_shifts, logit_weights,
                                             synthetic_image, window_shifts)

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]
DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _setup():
    oracle.build()
    yield
    torch.cuda.empty_cache()


def _case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _softplus_w(sh, B, C, H, W, seed, dtype, comp_box=True):
    g = torch.Generator().manual_seed(seed)
    w = torch.nn.functional.softplus(torch.randn(sh.size(0) * B, C, H, W, generator=g))
    if comp_box:
        w = w * box_stack(sh, B, H, W)
    return w.to(dtype)


# ---------------------------------------------------------------------------
# c0
# ---------------------------------------------------------------------------

def test_c0_accumulate_full_size():
    _case("c0 accumulate_uz fp32 256^2 R=3 comp_box")
    from test_golden import c0_golden
    x, w, sh, O = c0_golden()
    B, C, H, W = x.shape
    xd, wd = x.to(DEV).requires_grad_(True), w.to(DEV).requires_grad_(True)
    U, Z = accumulate_uz(xd, wd, sh.to(DEV))
    Us, Zs = oracle.accumulate_uz(x.abs(), w.abs(), sh)
    # the reference's CPU output (golden) and the fp64 oracle
    Uo, Zo = oracle.accumulate_uz(x, w, sh)
    assert_bound(U, Uo, Us, 1e-5, "U vs oracle")
    assert_bound(Z, Zo, Zs, 1e-5, "Z vs oracle")
    assert_bound(U, O["U"], Us, 2e-5, "U vs reference")
    assert_bound(Z, O["Z"], Zs, 2e-5, "Z vs reference")
    g = torch.Generator().manual_seed(3)
    gU = torch.randn(B, C, H, W, generator=g)
    gZ = torch.randn(B, C, H, W, generator=g)
    torch.autograd.backward([U, Z], [gU.to(DEV), gZ.to(DEV)])
    gxo, gwo = oracle.accumulate_uz_bwd(x, w, gU, gZ, sh)
    gxs, gws = oracle.accumulate_uz_bwd(x.abs(), w.abs(), gU.abs(), gZ.abs(), sh)
    assert_bound(xd.grad, gxo, gxs, 1e-5, "grad_x")
    assert_bound(wd.grad, gwo, gws, 1e-5, "grad_w")


# ---------------------------------------------------------------------------
# c1
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("mode", ["box", "periodic"])
def test_c1_gathers_bf16(mode):
    _case(f"c1 gathers {mode}")
    B, C, H, W = 8, 3, 256, 256
    sh = halfplane_shifts(5) if mode == "box" else window_shifts(5)
    guide = synthetic_image(B, C, H, W, seed=101).to(torch.bfloat16)
    gd = guide.to(DEV).requires_grad_(True)
    gs, mask = shift_gather(gd, sh.to(DEV))
    go, mo = oracle.shift_gather(guide, sh)
    assert torch.equal(gs.detach().cpu(), go) and torch.equal(mask.cpu(), mo)
    g = torch.Generator().manual_seed(5)
    gout = torch.randn(gs.shape, generator=g).to(torch.bfloat16)
    gs.backward(gout.to(DEV))
    ref = oracle.shift_gather_bwd(gout, sh, B, C, H, W)
    scale = oracle.shift_gather_bwd(gout.abs(), sh, B, C, H, W)
    assert_bound(gd.grad, ref, scale, 1e-5, "shift_gather grad", out_ulp_for(torch.bfloat16))
    del gs, mask, go, mo, gout
    gd.grad = None
    p, pm = pair_gather(gd, sh.to(DEV))
    po, pmo = oracle.pair_gather(guide, sh)
    assert torch.equal(p.detach().cpu(), po) and torch.equal(pm.cpu(), pmo)
    pout = torch.randn(p.shape, generator=g).to(torch.bfloat16)
    p.backward(pout.to(DEV))
    ref = oracle.pair_gather_bwd(pout, sh, B, C, H, W)
    scale = oracle.pair_gather_bwd(pout.abs(), sh, B, C, H, W)
    assert_bound(gd.grad, ref, scale, 1e-5, "pair_gather grad", out_ulp_for(torch.bfloat16))


# ---------------------------------------------------------------------------
# c2
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("weights", ["softplus", "logits"])
def test_c2_accumulate_fp16(weights):
    # "logits": the c2 weights as BASELINE.json gives them for the pair, N(0,
    # var 4) with 1% at +-80 -- signed, cancelling weights straight into
    # accumulate_uz (the scale of assert_bound is the sum of |terms|)
    _case(f"c2 accumulate_uz fp16 {weights}")
    B, C, H, W = 4, 1, 512, 512
    sh = halfplane_shifts(7)
    x = synthetic_image(B, C, H, W, seed=202).to(torch.float16)
    if weights == "softplus":
        w = _softplus_w(sh, B, C, H, W, 203, torch.float16)
    else:
        w = logit_weights((sh.size(0) * B, C, H, W), seed=203).to(torch.float16)
    g = torch.Generator().manual_seed(204)
    gU = torch.randn(B, C, H, W, generator=g)
    gZ = torch.randn(B, C, H, W, generator=g)
    xd, wd = x.to(DEV).requires_grad_(True), w.to(DEV).requires_grad_(True)
    U, Z = accumulate_uz(xd, wd, sh.to(DEV))
    torch.autograd.backward([U, Z], [gU.to(DEV), gZ.to(DEV)])
    Uo, Zo = oracle.accumulate_uz(x, w, sh)
    Us, Zs = oracle.accumulate_uz(x.abs(), w.abs(), sh)
    assert_bound(U, Uo, Us, 1e-5, "U")
    assert_bound(Z, Zo, Zs, 1e-5, "Z")
    del Uo, Zo, Us, Zs
    gxo, gwo = oracle.accumulate_uz_bwd(x, w, gU, gZ, sh)
    gxs, gws = oracle.accumulate_uz_bwd(x.abs(), w.abs(), gU.abs(), gZ.abs(), sh)
    ou = out_ulp_for(torch.float16)
    assert_bound(xd.grad, gxo, gxs, 1e-5, "grad_x", ou)
    assert_bound(wd.grad, gwo, gws, 1e-5, "grad_w", ou)


def test_c2_normalized_log_weights_fp16():
    _case("c2 normalized fp16 log weights")
    B, C, H, W = 4, 1, 512, 512
    sh = halfplane_shifts(7)
    x = synthetic_image(B, C, H, W, seed=205).to(torch.float16)
    lw = logit_weights((sh.size(0) * B, C, H, W), seed=206).to(torch.float16)
    g = torch.Generator().manual_seed(207)
    gD = torch.randn(B, C, H, W, generator=g)
    gL = torch.randn(B, C, H, W, generator=g)
    xd, wd = x.to(DEV).requires_grad_(True), lw.to(DEV).requires_grad_(True)
    D, L = normalized_accumulate_uz(xd, wd, sh.to(DEV), log_weights=True, return_log_degree=True)
    torch.autograd.backward([D, L], [gD.to(DEV), gL.to(DEV)])
    Do, Lo = oracle.normalized(x, lw, sh, log_weights=True, policy="gpu")
    Ds, _ = oracle.normalized(x.abs(), lw, sh, log_weights=True, policy="gpu")
    assert_bound(D, Do, Ds, 1e-5, "D")
    assert_bound(L, Lo, Lo.abs() + 1.0, 1e-5, "log_C")
    gxo, gwo = oracle.normalized_bwd(x, lw, Do, Lo, gD, gL, sh, log_weights=True)
    # x[p+s] - D enters each weight gradient: D's own error (<= rtol * Ds) propagates,
    # so the scale takes Ds = sum w|x| / C >= |D| in D's place
    gxs, gws = oracle.normalized_bwd(x.abs(), lw, -Ds, Lo, gD.abs(), gL.abs(), sh,
                                     log_weights=True)
    ou = out_ulp_for(torch.float16)
    # the fractions exp(l - log C) carry the forward's log C error and the
    # |l - log C| conditioning (up to ~160 with +-80 logits): derived per term
    gxc, gwc = normalized_bwd_cond(x, lw, Lo, gD, gL, Ds, sh, log_weights=True,
                                   acc_dtype=torch.float16)
    assert_bound(xd.grad, gxo, gxs, 1e-5, "grad_x", ou, extra=gxc)
    assert_bound(wd.grad, gwo, gws, 1e-5, "grad_w", ou, extra=gwc)


# ---------------------------------------------------------------------------
# c3
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype,B,comp_box", [(torch.float32, 16, True),
                                              (torch.float32, 16, False),
                                              (torch.float64, 2, True)])
def test_c3_gasd_full_window(dtype, B, comp_box):
    _case(f"c3 GASD {dtype} B={B} comp_box={comp_box}")
    C, H, W = 3, 256, 256
    sh = window_shifts(5)
    x = synthetic_image(B, C, H, W, seed=301).to(dtype)
    w = _softplus_w(sh, B, C, H, W, 302, dtype, comp_box)
    g = torch.Generator().manual_seed(303)
    gU = torch.randn(B, C, H, W, generator=g, dtype=dtype)
    gZ = torch.randn(B, C, H, W, generator=g, dtype=dtype)
    rt = rtol_for(dtype)
    xd, wd = x.to(DEV).requires_grad_(True), w.to(DEV).requires_grad_(True)
    U, Z = accumulate_uz(xd, wd, sh.to(DEV))
    torch.autograd.backward([U, Z], [gU.to(DEV), gZ.to(DEV)])
    Uo, Zo = oracle.accumulate_uz(x, w, sh)
    Us, Zs = oracle.accumulate_uz(x.abs(), w.abs(), sh)
    assert_bound(U, Uo, Us, rt, "U")
    assert_bound(Z, Zo, Zs, rt, "Z")
    del Us, Zs
    gxo, gwo = oracle.accumulate_uz_bwd(x, w, gU, gZ, sh)
    gxs, gws = oracle.accumulate_uz_bwd(x.abs(), w.abs(), gU.abs(), gZ.abs(), sh)
    assert_bound(xd.grad, gxo, gxs, rt, "grad_x")
    assert_bound(wd.grad, gwo, gws, rt, "grad_w")
    del gxo, gwo, gxs, gws
    # row-stochastic Z^-1 U through the normalized op (positive weights)
    xd.grad = None
    wd.grad = None
    D = normalized_accumulate_uz(xd, wd, sh.to(DEV), validate=False)
    D.backward(gU.to(DEV))
    Do, Lo = oracle.normalized(x, w, sh, log_weights=False, policy="gpu")
    Ds, _ = oracle.normalized(x.abs(), w, sh, log_weights=False, policy="gpu")
    assert_bound(D, Do, Ds, rt, "D")
    assert torch.allclose(Do, Uo / Zo, rtol=1e-12, atol=1e-12)  # D is Z^-1 U
    gxo, gwo = oracle.normalized_bwd(x, w, Do, Lo, gU, torch.zeros_like(gU), sh, log_weights=False)
    # x[p+s] - D enters each weight gradient: D's own error (<= rtol * Ds) propagates,
    # so the scale takes Ds = sum w|x| / C >= |D| in D's place
    gxs, gws = oracle.normalized_bwd(x.abs(), w, -Ds, Lo, gU.abs(), torch.zeros_like(gU), sh,
                                     log_weights=False)
    gxc, gwc = normalized_bwd_cond(x, w, Lo, gU, torch.zeros_like(gU), Ds, sh,
                                   log_weights=False, acc_dtype=dtype)
    assert_bound(xd.grad, gxo, gxs, rt, "D grad_x", extra=gxc)
    assert_bound(wd.grad, gwo, gws, rt, "D grad_w", extra=gwc)


# ---------------------------------------------------------------------------
# c4
# ---------------------------------------------------------------------------

C4 = (1, 1, 8192, 8192, 6)


def _c4_inputs(seed):
    B, C, H, W, R = C4
    sh = halfplane_shifts(R)
    S = sh.size(0)
    x = synthetic_image(B, C, H, W, seed=seed).to(DEV)
    w = torch.empty(S * B, C, H, W, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(seed + 1)
    for s in range(S):
        blk = torch.nn.functional.softplus(torch.randn(B, C, H, W, generator=g, device=DEV))
        w[s * B:(s + 1) * B] = blk * box_stack(sh[s:s + 1], 1, H, W, device=DEV)
    return x, w, sh


def _crops(n, H, W, ch, cw, seed):
    g = torch.Generator().manual_seed(seed)
    out = [(0, 0), (H - ch, W - cw), (0, W - cw // 2), (H - ch // 2, 3)]  # borders + wraps
    while len(out) < n:
        out.append((int(torch.randint(0, H, (1,), generator=g)), int(torch.randint(0, W, (1,), generator=g))))
    return out


def test_c4_accumulate_int64_stress_crops():
    _case("c4 accumulate_uz fwd+bwd 8192^2 S=85")
    B, C, H, W, R = C4
    x, w, sh = _c4_inputs(401)
    S = sh.size(0)
    assert S * B * C * H * W > 2 ** 31
    g = torch.Generator(device=DEV).manual_seed(403)
    gU = torch.randn(B, C, H, W, generator=g, device=DEV)
    gZ = torch.randn(B, C, H, W, generator=g, device=DEV)
    x.requires_grad_(True)
    w.requires_grad_(True)
    U, Z = accumulate_uz(x, w, sh.to(DEV))
    torch.autograd.backward([U, Z], [gU, gZ])
    ch = cw = 256
    halo = R
    xs, ws, gUd, gZd = x.detach(), w.detach(), gU, gZ
    for k, (gh0, gw0) in enumerate(_crops(64, H, W, ch, cw, 404)):
        win = lambda t: oracle.take_window(t, gh0, gw0, ch, cw, halo)
        crop = lambda t: oracle.take_window(t, gh0, gw0, ch, cw, 0)
        xw, ww = win(xs), win(ws)
        Uo, Zo = oracle.accumulate_uz_window(xw, ww, sh, halo, H, W, gh0, gw0, ch, cw)
        Us, Zs = oracle.accumulate_uz_window(xw.abs(), ww.abs(), sh, halo, H, W, gh0, gw0, ch, cw)
        assert_bound(crop(U.detach()), Uo, Us, 1e-5, f"U crop {k} at {(gh0, gw0)}")
        assert_bound(crop(Z.detach()), Zo, Zs, 1e-5, f"Z crop {k} at {(gh0, gw0)}")
        gUw, gZw = win(gUd), win(gZd)
        gxo, gwo = oracle.accumulate_uz_window_bwd(xw, ww, gUw, gZw, sh, halo, H, W, gh0, gw0, ch, cw)
        gxs, gws = oracle.accumulate_uz_window_bwd(xw.abs(), ww.abs(), gUw.abs(), gZw.abs(), sh,
                                                   halo, H, W, gh0, gw0, ch, cw)
        assert_bound(crop(x.grad), gxo, gxs, 1e-5, f"grad_x crop {k}")
        assert_bound(crop(w.grad), gwo, gws, 1e-5, f"grad_w crop {k}")
    del x, w, U, Z, gU, gZ
    torch.cuda.empty_cache()


def test_c4_metropolis_symmetry_and_crops():
    _case("c4 metropolis 8192^2 S=85")
    B, C, H, W, R = C4
    sh = halfplane_shifts(R)
    S = sh.size(0)
    shifts = [(dx, dy, bool(inv)) for dx, dy, inv in sh.tolist()]
    img = synthetic_image(B, C, H, W, seed=501).to(DEV)
    wh = torch.empty(B, S, C, H, W, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(502)
    for s in range(S):
        wh[:, s] = torch.nn.functional.softplus(torch.randn(B, C, H, W, generator=g, device=DEV))
    with torch.no_grad():
        Wx, dh = metropolis_aggregate(wh, img, shifts, True)
        ch = cw = 256
        halo = 2 * R
        for k, (gh0, gw0) in enumerate(_crops(64, H, W, ch, cw, 503)):
            whw = oracle.take_window(wh, gh0, gw0, ch, cw, halo)
            imw = oracle.take_window(img, gh0, gw0, ch, cw, halo)
            Wo, do = oracle.metropolis_window(whw, imw, sh, halo, H, W, gh0, gw0, ch, cw, True)
            Ws, _ = oracle.metropolis_window(whw, imw.abs(), sh, halo, H, W, gh0, gw0, ch, cw, True)
            crop = lambda t: oracle.take_window(t, gh0, gw0, ch, cw, 0)
            scale = Ws.abs() + 2 * crop(img).double().abs() * (1 + do.abs())
            assert_bound(crop(Wx), Wo, scale, 1e-5, f"Wx crop {k}")
            assert_bound(crop(dh), do, do.abs(), 1e-5, f"d_hat crop {k}")
        del Wx, dh
        # exact symmetry (W e_j)_i == (W e_i)_j for sampled neighbour pairs
        pairs = [((100, 200), (103, 204)), ((0, 0), (2, 8191)), ((8191, 5), (8186, 0)),
                 ((4000, 4000), (4006, 4001)), ((7, 7), (7, 8))]
        for i, j in pairs:
            ei = torch.zeros(B, C, H, W, device=DEV)
            ej = torch.zeros(B, C, H, W, device=DEV)
            ei[0, 0, i[0], i[1]] = 1.0
            ej[0, 0, j[0], j[1]] = 1.0
            Wej, _ = metropolis_aggregate(wh, ej, shifts, True)
            Wei, _ = metropolis_aggregate(wh, ei, shifts, True)
            a = Wej[0, 0, i[0], i[1]].item()
            b = Wei[0, 0, j[0], j[1]].item()
            assert a == b, f"W not symmetric at {i},{j}: {a} vs {b}"
            del Wej, Wei
    del wh, img
    torch.cuda.empty_cache()
