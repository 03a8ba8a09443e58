"""Pins of the CPU oracle (oracle/oracle.c) -- runs on the CPU.

Each oracle function is checked against something that does not share its
formulation, chosen so that a plausible mistake (dropped mirror term, wrong
shift sign, box on the wrong side, circular vs non-circular mirror, missing
gZ term, wrong normalisation) fails:

* dense operator matrices assembled pixel by pixel (tests/helpers.py) and
  torch autograd through them (gradients);
* torch.roll closed forms, as the reference's own test fixture
  ``_symmetric_serial`` (tests/test_cached_forward_patches.py:34-49) writes
  the operator;
* the reference's CPU known-answer tests
  (tests/test_normalized_accumulate_uz.py:30-81) restated against the oracle;
* mathematical invariants: adjointness, exact symmetry and row
  stochasticity of the Metropolis W, offset invariance of log weights;
* golden vectors produced by the reference's CPU fallback
  (tests/golden/, when present).
"""
from __future__ import annotations

import itertools

import pytest
import torch

import oracle
from helpers import (assert_bound, box_np, dense_accumulate, dense_metropolis,
                     dense_normalized, roll_gather)
from neural_shift_cuda_amd.workloads import (explicit_mirror_shifts, halfplane_shifts,
                                             window_shifts)

pytestmark = pytest.mark.filterwarnings("ignore::UserWarning")


@pytest.fixture(scope="module", autouse=True)
def _build_oracle():
    oracle.build()


def _tables():
    return {
        "half1": halfplane_shifts(1),
        "half2": halfplane_shifts(2),
        "win1": window_shifts(1),
        "mirror2": explicit_mirror_shifts(halfplane_shifts(2)),
        "odd": torch.tensor([[0, 0, 0], [3, -2, 1], [-1, 4, 1], [2, 0, 0]]),
    }


# ---------------------------------------------------------------------------
# gathers
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("name", ["half2", "win1", "odd"])
def test_gather_matches_roll_and_box(dtype, name):
    sh = _tables()[name]
    g = torch.Generator().manual_seed(0)
    guide = torch.randn(2, 3, 7, 9, generator=g).to(dtype)
    gs, mask = oracle.shift_gather(guide, sh)
    pair, pmask = oracle.pair_gather(guide, sh)
    B = guide.size(0)
    for s, (dx, dy) in enumerate(sh[:, :2].tolist()):
        exp = roll_gather(guide, dx, dy)
        assert torch.equal(gs[s * B:(s + 1) * B].view(torch.int16 if dtype.itemsize == 2 else dtype),
                           exp.view(torch.int16 if dtype.itemsize == 2 else dtype))
        assert torch.equal(pair[s * B:(s + 1) * B, :3], guide)
        assert torch.equal(pair[s * B:(s + 1) * B, 3:], exp)
        m = box_np(7, 9, dx, dy).to(dtype)
        assert torch.equal(mask[s * B:(s + 1) * B, 0], m.expand(B, 7, 9))
        assert torch.equal(pmask, mask)


def test_gather_zero_radius_all_ones_mask():
    # the reference's R == 0 branch (ops.py:112-116): repeat + all-ones mask
    guide = torch.randn(2, 2, 4, 5)
    sh = torch.zeros(3, 2, dtype=torch.int64)
    gs, mask = oracle.shift_gather(guide, sh)
    assert torch.equal(gs, guide.repeat(3, 1, 1, 1))
    assert torch.equal(mask, torch.ones(6, 1, 4, 5))


@pytest.mark.parametrize("pair", [False, True])
def test_gather_backward_is_adjoint(pair):
    sh = _tables()["odd"]
    g = torch.Generator().manual_seed(1)
    guide = torch.randn(2, 2, 6, 5, dtype=torch.float64, generator=g, requires_grad=True)
    ref = []
    for dx, dy in sh[:, :2].tolist():
        ref.append(roll_gather(guide, dx, dy))
    out = torch.cat(ref, 0)
    if pair:
        out = torch.cat((guide.repeat(len(ref), 1, 1, 1), out), 1)
    gout = torch.randn(out.shape, dtype=torch.float64, generator=g)
    (out * gout).sum().backward()
    fn = oracle.pair_gather_bwd if pair else oracle.shift_gather_bwd
    got = fn(gout, sh, 2, 2, 6, 5)
    assert torch.allclose(got, guide.grad, rtol=0, atol=1e-13)


# ---------------------------------------------------------------------------
# accumulate_uz
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["half1", "half2", "win1", "mirror2", "odd"])
def test_accumulate_matches_dense_operator(name):
    sh = _tables()[name]
    B, C, H, W = 2, 2, 6, 7
    g = torch.Generator().manual_seed(2)
    x = torch.randn(B, C, H, W, dtype=torch.float64, generator=g)
    w = torch.randn(sh.size(0) * B, C, H, W, dtype=torch.float64, generator=g)
    U, Z = oracle.accumulate_uz(x, w, sh)
    Ud, Zd = dense_accumulate(x, w, sh.tolist())
    assert torch.allclose(U, Ud, rtol=1e-12, atol=1e-12)
    assert torch.allclose(Z, Zd, rtol=1e-12, atol=1e-12)


def test_accumulate_matches_symmetric_serial_closed_form():
    # _symmetric_serial (reference tests/test_cached_forward_patches.py:34-49)
    sh = halfplane_shifts(2)
    B, C, H, W = 2, 3, 7, 8
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, C, H, W, dtype=torch.float64, generator=g)
    w = torch.rand(sh.size(0) * B, C, H, W, dtype=torch.float64, generator=g)
    U = torch.zeros_like(x)
    Z = torch.zeros_like(x)
    for s, (dx, dy, inv) in enumerate(sh.tolist()):
        wf = w[s * B:(s + 1) * B]
        U = U + wf * roll_gather(x, dx, dy)
        Z = Z + wf
        if inv:
            wi = torch.roll(wf, shifts=(dx, dy), dims=(-2, -1)) * box_np(H, W, -dx, -dy)
            U = U + wi * roll_gather(x, -dx, -dy)
            Z = Z + wi
    Uo, Zo = oracle.accumulate_uz(x, w, sh)
    assert torch.allclose(Uo, U, rtol=1e-12, atol=1e-12)
    assert torch.allclose(Zo, Z, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("name", ["half2", "win1", "odd"])
def test_accumulate_backward_matches_autograd_of_dense(name):
    sh = _tables()[name]
    B, C, H, W = 2, 2, 5, 6
    g = torch.Generator().manual_seed(4)
    x = torch.randn(B, C, H, W, dtype=torch.float64, generator=g, requires_grad=True)
    w = torch.randn(sh.size(0) * B, C, H, W, dtype=torch.float64, generator=g,
                    requires_grad=True)
    gU = torch.randn(B, C, H, W, dtype=torch.float64, generator=g)
    gZ = torch.randn(B, C, H, W, dtype=torch.float64, generator=g)
    U, Z = dense_accumulate(x, w, sh.tolist())
    (U * gU + Z * gZ).sum().backward()
    gx, gw = oracle.accumulate_uz_bwd(x, w, gU, gZ, sh)
    assert torch.allclose(gx, x.grad, rtol=1e-12, atol=1e-12)
    assert torch.allclose(gw, w.grad, rtol=1e-12, atol=1e-12)


def test_accumulate_float_mode_is_tree_ordered_float_arithmetic():
    # float mode must equal the same tree evaluated in float on the fp64 terms
    # rounded per operation -- checked against the fp64 result within the
    # tree's error bound, and to differ from naive serial float summation in
    # at least one element for a cancellation-heavy input.
    sh = halfplane_shifts(3)
    B, C, H, W = 1, 1, 16, 16
    g = torch.Generator().manual_seed(5)
    x = torch.randn(B, C, H, W, generator=g)
    w = torch.randn(sh.size(0) * B, C, H, W, generator=g) * 1e3
    U32, _ = oracle.accumulate_uz(x, w, sh, dtype=torch.float32)
    U64, _ = oracle.accumulate_uz(x, w, sh, dtype=torch.float64)
    Us, _ = oracle.accumulate_uz(x.abs(), w.abs(), sh, dtype=torch.float64)
    assert_bound(U32, U64, Us, rtol=8 * 2.0 ** -23, what="fp32 tree")


# ---------------------------------------------------------------------------
# normalized_accumulate_uz
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("policy", ["cpu", "gpu"])
@pytest.mark.parametrize("log_weights", [False, True])
@pytest.mark.parametrize("name", ["half2", "win1", "odd"])
def test_normalized_matches_dense_softmax(policy, log_weights, name):
    sh = _tables()[name]
    B, C, H, W = 1, 2, 6, 5
    g = torch.Generator().manual_seed(6)
    x = torch.randn(B, C, H, W, dtype=torch.float64, generator=g)
    raw = torch.randn(sh.size(0) * B, C, H, W, dtype=torch.float64, generator=g)
    w = raw * 3 if log_weights else raw.exp()
    # masks: some -inf logits / zero weights, one fully masked pixel row
    m = torch.rand(w.shape, generator=g) < 0.2
    w = torch.where(m, torch.full_like(w, float("-inf") if log_weights else 0.0), w)
    D, L = oracle.normalized(x, w, sh, log_weights=log_weights, policy=policy)
    Dd, Ld = dense_normalized(x, w, sh.tolist(), log_weights)
    assert torch.allclose(D, Dd, rtol=1e-12, atol=1e-12)
    assert torch.allclose(L, Ld, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("log_weights", [False, True])
def test_normalized_empty_rows(log_weights):
    sh = window_shifts(1)
    x = torch.randn(1, 1, 4, 4, dtype=torch.float64)
    w = torch.full((9, 1, 4, 4), float("-inf") if log_weights else 0.0, dtype=torch.float64)
    w[:, :, 0, 0] = 1.0  # only pixel (0,0) has terms
    for policy in ("cpu", "gpu"):
        D, L = oracle.normalized(x, w, sh, log_weights=log_weights, policy=policy)
        assert D[0, 0, 0, 0] != 0
        assert torch.all(D.flatten()[1:] == 0)
        assert torch.all(torch.isneginf(L.flatten()[1:]))


def test_normalized_negative_weight_policy():
    # reference CPU fallback masks a negative positive-mode weight
    # (ops.py:227-231); the reference GPU kernel propagates NaN
    # (shift_ops_cuda.cu:498-503).
    sh = window_shifts(1)
    x = torch.randn(1, 1, 4, 4, dtype=torch.float64)
    w = torch.rand(9, 1, 4, 4, dtype=torch.float64) + 0.1
    w[3, 0, 2, 2] = -1.0
    Dc, _ = oracle.normalized(x, w, sh, log_weights=False, policy="cpu")
    Dg, Lg = oracle.normalized(x, w, sh, log_weights=False, policy="gpu")
    assert torch.isfinite(Dc).all()
    assert torch.isnan(Dg[0, 0, 2, 2]) and torch.isnan(Lg[0, 0, 2, 2])
    assert torch.isfinite(Dg).sum() == 15


def test_normalized_stable_equals_exact_ratio():
    # reference tests/test_normalized_accumulate_uz.py:30-40
    sh = halfplane_shifts(2)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 3, 7, 6, dtype=torch.float64, generator=g)
    w = torch.rand(sh.size(0) * 2, 3, 7, 6, dtype=torch.float64, generator=g) + 0.1
    U, Z = oracle.accumulate_uz(x, w, sh)
    for policy in ("cpu", "gpu"):
        D, L = oracle.normalized(x, w, sh, log_weights=False, policy=policy)
        assert torch.allclose(D, U / Z, rtol=1e-12, atol=1e-12)
        assert torch.allclose(L, Z.log(), rtol=1e-12, atol=1e-12)


def test_normalized_overflow_closed_form_fp32():
    # reference tests/test_normalized_accumulate_uz.py:43-61: uniform 1e38
    # weights overflow the unscaled degree but D is the mean of the 9 rolls.
    sh = window_shifts(1)
    x = torch.linspace(-1, 1, 20).reshape(1, 1, 5, 4)
    w = torch.full((9, 1, 5, 4), 1.0e38)
    exp = torch.stack([roll_gather(x, dx, dy) for dx, dy, _ in sh.tolist()]).mean(0)
    for policy in ("cpu", "gpu"):
        D, L = oracle.normalized(x, w, sh, log_weights=False, policy=policy,
                                 dtype=torch.float32)
        assert torch.isfinite(D).all() and torch.isfinite(L).all()
        assert torch.allclose(D, exp, rtol=2e-6, atol=2e-6)
        assert torch.allclose(L, torch.full_like(L, float(torch.tensor(9e38, dtype=torch.float64).log())),
                              rtol=1e-6)


def test_normalized_log_offset_invariance():
    # reference tests/test_normalized_accumulate_uz.py:64-81
    sh = window_shifts(2)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, 2, 6, 5, generator=g)
    logits = 10_000.0 + 3.0 * torch.randn(25, 2, 6, 5, generator=g)
    d1, l1 = oracle.normalized(x, logits, sh, log_weights=True, dtype=torch.float32)
    d2, l2 = oracle.normalized(x, logits + 5_000.0, sh, log_weights=True, dtype=torch.float32)
    assert torch.isfinite(d1).all()
    assert torch.allclose(d1, d2, rtol=2e-5, atol=2e-5)
    assert torch.allclose(l2 - l1, torch.full_like(l1, 5_000.0), rtol=0, atol=2e-3)


@pytest.mark.parametrize("log_weights", [False, True])
@pytest.mark.parametrize("name", ["half2", "win1"])
def test_normalized_backward_matches_autograd_of_dense(log_weights, name):
    sh = _tables()[name]
    B, C, H, W = 1, 2, 5, 6
    g = torch.Generator().manual_seed(7)
    x = torch.randn(B, C, H, W, dtype=torch.float64, generator=g, requires_grad=True)
    raw = torch.randn(sh.size(0) * B, C, H, W, dtype=torch.float64, generator=g)
    w0 = raw if log_weights else raw.exp()
    m = torch.rand(w0.shape, generator=g) < 0.15
    w0 = torch.where(m, torch.full_like(w0, float("-inf") if log_weights else 0.0), w0)
    w = w0.clone().requires_grad_(True)
    gD = torch.randn(B, C, H, W, dtype=torch.float64, generator=g)
    gL = torch.randn(B, C, H, W, dtype=torch.float64, generator=g)
    D, L = dense_normalized(x, w, sh.tolist(), log_weights)
    (D * gD + L * gL).sum().backward()
    gx, gw = oracle.normalized_bwd(x, w0, D.detach(), L.detach(), gD, gL, sh,
                                   log_weights=log_weights)
    assert torch.allclose(gx, x.grad, rtol=1e-10, atol=1e-11)
    # masked weights: the reference GPU rule is a zero gradient
    assert torch.all(gw[m] == 0)
    assert torch.allclose(gw[~m], w.grad[~m], rtol=1e-10, atol=1e-11)


# ---------------------------------------------------------------------------
# Metropolis
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("use_box", [True, False])
def test_metropolis_matches_dense_and_is_symmetric_stochastic(use_box):
    sh = halfplane_shifts(1)
    B, S, C, H, W = 1, sh.size(0), 2, 5, 6
    g = torch.Generator().manual_seed(8)
    wh = torch.nn.functional.softplus(torch.randn(B, S, C, H, W, dtype=torch.float64, generator=g))
    img = torch.randn(B, C, H, W, dtype=torch.float64, generator=g)
    Wx, dh = oracle.metropolis(wh, img, sh, use_box, eps=1e-6)
    Wd, dd, mats = dense_metropolis(wh, img, sh.tolist(), use_box, 1e-6)
    assert torch.allclose(Wx, Wd, rtol=1e-12, atol=1e-12)
    assert torch.allclose(dh, dd, rtol=1e-12, atol=1e-12)
    for Wm in mats:
        assert torch.allclose(Wm, Wm.T, rtol=0, atol=1e-15)
        assert torch.allclose(Wm.sum(1), torch.ones(H * W, dtype=torch.float64), atol=1e-12)


@pytest.mark.parametrize("use_box", [True, False])
def test_metropolis_ordered_reference_is_the_operator(use_box):
    """helpers.metropolis_torch_ordered (the GPU backward tests' reference)
    with the exact degree as its ordering is the operator itself: the C
    oracle's values and the gradients of plain autograd through
    metropolis_aggregate_torch, torch.maximum's tie split included (the
    (0, 0, 1) row is a self edge, an exact tie at every pixel).  Flipping
    one edge's ordering moves the value by at most |d_p - d_j| / m times
    that edge's terms."""
    from helpers import metropolis_torch_ordered
    from neural_shift_cuda_amd.metropolis import metropolis_aggregate_torch
    rows = [(0, 0, True), (1, 0, True), (0, 1, True), (-1, 2, False), (2, -1, True)]
    B, S, C, H, W = 1, len(rows), 2, 6, 7
    g = torch.Generator().manual_seed(12)
    wh = torch.nn.functional.softplus(torch.randn(B, S, C, H, W, dtype=torch.float64, generator=g))
    img = torch.randn(B, C, H, W, dtype=torch.float64, generator=g)
    gW = torch.randn(B, C, H, W, dtype=torch.float64, generator=g)
    gd = torch.randn(B, C, H, W, dtype=torch.float64, generator=g)
    sh = torch.tensor([[dx, dy, int(i)] for dx, dy, i in rows])
    d = torch.zeros(B, C, H, W, dtype=torch.float64)
    for s, (dx, dy, inv) in enumerate(rows):
        o = wh[:, s] * (box_np(H, W, dx, dy) if use_box else 1.0)
        d = d + o + (torch.roll(o, (dx, dy), (-2, -1)) if inv else 0)
    grads = []
    for fn in (lambda w, x: metropolis_torch_ordered(w, x, rows, use_box, d),
               lambda w, x: metropolis_aggregate_torch(w, x, rows, use_box)):
        w = wh.clone().requires_grad_(True)
        x = img.clone().requires_grad_(True)
        Wx, dh = fn(w, x)
        torch.autograd.backward([Wx, dh], [gW, gd])
        grads.append((Wx.detach(), dh.detach(), w.grad, x.grad))
    Wo, do = oracle.metropolis(wh, img, sh, use_box)
    assert torch.allclose(grads[0][0], Wo, rtol=1e-13, atol=1e-13)
    assert torch.allclose(grads[0][1], do, rtol=1e-13, atol=1e-13)
    for a, b in zip(grads[0], grads[1]):
        assert torch.allclose(a, b, rtol=1e-13, atol=1e-13)


def test_metropolis_exact_symmetry_basis_vectors():
    # (W e_j)_i == (W e_i)_j bit for bit, fp32 oracle
    sh = halfplane_shifts(2)
    B, S, C, H, W = 1, sh.size(0), 1, 8, 9
    g = torch.Generator().manual_seed(9)
    wh = torch.nn.functional.softplus(torch.randn(B, S, C, H, W, generator=g))
    pairs = [((1, 2), (2, 3)), ((0, 0), (1, 8)), ((4, 4), (6, 5)), ((7, 8), (7, 7))]
    for (i, j) in pairs:
        ei = torch.zeros(B, C, H, W)
        ej = torch.zeros(B, C, H, W)
        ei[0, 0, i[0], i[1]] = 1
        ej[0, 0, j[0], j[1]] = 1
        Wej, _ = oracle.metropolis(wh, ej, sh, True, dtype=torch.float32)
        Wei, _ = oracle.metropolis(wh, ei, sh, True, dtype=torch.float32)
        assert Wej[0, 0, i[0], i[1]].item() == Wei[0, 0, j[0], j[1]].item()


# ---------------------------------------------------------------------------
# accumulate_uz_scalar
# ---------------------------------------------------------------------------

def test_scalar_matches_roll_and_autograd():
    sh = window_shifts(2, with_flag=False)
    B, C, H, W = 2, 3, 7, 6
    g = torch.Generator().manual_seed(10)
    x = torch.randn(B, C, H, W, dtype=torch.float64, generator=g, requires_grad=True)
    w = (torch.rand(sh.size(0), B, C, dtype=torch.float64, generator=g) + 0.1).requires_grad_(True)
    U = sum(w[s].reshape(B, C, 1, 1) * roll_gather(x, dx, dy)
            for s, (dx, dy) in enumerate(sh.tolist()))
    Z = w.sum(0).reshape(B, C, 1, 1).expand(B, C, H, W)
    Uo, Zo = oracle.accumulate_uz_scalar(x, w, sh)
    assert torch.allclose(Uo, U, rtol=1e-12, atol=1e-12)
    assert torch.allclose(Zo, Z, rtol=1e-12, atol=1e-12)
    gU = torch.randn(B, C, H, W, dtype=torch.float64, generator=g)
    gZ = torch.randn(B, C, H, W, dtype=torch.float64, generator=g)
    (U * gU + Z * gZ).sum().backward()
    gx, gw = oracle.accumulate_uz_scalar_bwd(x, w, gU, gZ, sh)
    assert torch.allclose(gx, x.grad, rtol=1e-12, atol=1e-12)
    assert torch.allclose(gw, w.grad, rtol=1e-12, atol=1e-11)


# ---------------------------------------------------------------------------
# window evaluation == full-image evaluation on the crop (bit for bit)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("crop", [(0, 0), (13, 7), (30, 41), (35, 45), (20, 0)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_window_oracle_equals_full(crop, dtype):
    sh = halfplane_shifts(3)
    B, C, H, W = 1, 2, 40, 50
    ch, cw, halo = 9, 11, 6
    gh0, gw0 = crop
    g = torch.Generator().manual_seed(12)
    x = torch.randn(B, C, H, W, dtype=dtype, generator=g)
    w = torch.randn(sh.size(0) * B, C, H, W, dtype=dtype, generator=g)
    gU = torch.randn(B, C, H, W, dtype=dtype, generator=g)
    gZ = torch.randn(B, C, H, W, dtype=dtype, generator=g)
    U, Z = oracle.accumulate_uz(x, w, sh, dtype=dtype)
    gx, gw = oracle.accumulate_uz_bwd(x, w, gU, gZ, sh, dtype=dtype)
    rows = oracle.window_indices(H, gh0, 0, ch)
    cols = oracle.window_indices(W, gw0, 0, cw)
    crop_of = lambda t: t.index_select(-2, rows).index_select(-1, cols)
    win = lambda t: oracle.take_window(t, gh0, gw0, ch, cw, halo)
    Uw, Zw = oracle.accumulate_uz_window(win(x), win(w), sh, halo, H, W, gh0, gw0, ch, cw,
                                         dtype=dtype)
    assert torch.equal(Uw, crop_of(U)) and torch.equal(Zw, crop_of(Z))
    gxw, gww = oracle.accumulate_uz_window_bwd(win(x), win(w), win(gU), win(gZ), sh, halo, H, W,
                                               gh0, gw0, ch, cw, dtype=dtype)
    assert torch.equal(gxw, crop_of(gx)) and torch.equal(gww, crop_of(gw))
    for use_box in (True, False):
        wh = torch.nn.functional.softplus(
            torch.randn(B, sh.size(0), C, H, W, dtype=dtype, generator=g))
        Wx, dh = oracle.metropolis(wh, x, sh, use_box, dtype=dtype)
        Wxw, dhw = oracle.metropolis_window(oracle.take_window(wh, gh0, gw0, ch, cw, 2 * halo),
                                            oracle.take_window(x, gh0, gw0, ch, cw, 2 * halo),
                                            sh, 2 * halo, H, W, gh0, gw0, ch, cw, use_box,
                                            dtype=dtype)
        assert torch.equal(Wxw, crop_of(Wx)) and torch.equal(dhw, crop_of(dh))
