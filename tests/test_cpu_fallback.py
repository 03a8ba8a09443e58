"""The package's PyTorch CPU fallbacks (the ``*_reference`` functions and the
CPU dispatch of the public ops) against the oracle, plus the reference's CPU
known-answer, gradcheck, promotion and validation tests restated
(reference tests/test_normalized_accumulate_uz.py, test_index_width.py,
test_accumulate_uz_scalar.py:39-79)."""
from __future__ import annotations

import pytest
import torch

import oracle
from helpers import assert_bound, roll_gather
from neural_shift_cuda import (accumulate_uz, accumulate_uz_reference, accumulate_uz_scalar,
                               accumulate_uz_scalar_reference, metropolis_aggregate,
                               normalized_accumulate_uz, normalized_accumulate_uz_reference,
                               pair_gather, pair_gather_reference, shift_gather,
                               shift_gather_reference)
from neural_shift_cuda.metropolis import metropolis_aggregate_fused, metropolis_aggregate_torch
from neural_shift_cuda.ops import _prep_shifts_for_cuda
from neural_shift_cuda_amd.workloads import (box_stack, explicit_mirror_shifts, halfplane_shifts,
                                             window_shifts)


@pytest.fixture(scope="module", autouse=True)
def _build_oracle():
    oracle.build()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("R", [0, 1, 2, 5])
def test_gathers_bit_exact_vs_oracle(dtype, R):
    guide = torch.randn(2, 3, 13, 11).to(dtype)
    sh = halfplane_shifts(R)
    gs, m = shift_gather(guide, sh)
    go, mo = oracle.shift_gather(guide, sh)
    assert gs.dtype == dtype and m.dtype == dtype
    assert torch.equal(gs, go) and torch.equal(m, mo)
    p, pm = pair_gather(guide, sh)
    po, pmo = oracle.pair_gather(guide, sh)
    assert torch.equal(p, po) and torch.equal(pm, pmo)


@pytest.mark.parametrize("shape", [(1, 3, 16, 16), (2, 3, 31, 29), (3, 2, 33, 47)])
@pytest.mark.parametrize("R", [1, 2, 4])
def test_accumulate_fp32_bit_exact_vs_oracle_tree(shape, R):
    # both restate the reference term order and pairwise tree
    B, C, H, W = shape
    sh = halfplane_shifts(R)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, C, H, W, generator=g)
    w = torch.randn(sh.size(0) * B, C, H, W, generator=g) * box_stack(sh, B, H, W)
    U, Z = accumulate_uz(x, w, sh)
    Uo, Zo = oracle.accumulate_uz(x, w, sh, dtype=torch.float32)
    assert torch.equal(U, Uo) and torch.equal(Z, Zo)


def test_accumulate_fp64_gradients_vs_oracle():
    sh = halfplane_shifts(3)
    B, C, H, W = 2, 3, 13, 11
    g = torch.Generator().manual_seed(7)
    x = torch.randn(B, C, H, W, dtype=torch.float64, generator=g, requires_grad=True)
    w = (torch.randn(sh.size(0) * B, C, H, W, dtype=torch.float64, generator=g)
         * box_stack(sh, B, H, W, torch.float64)).requires_grad_(True)
    U, Z = accumulate_uz_reference(x, w, sh)
    gU = torch.randn_like(U)
    gZ = torch.randn_like(Z)
    (U * gU + Z * gZ).sum().backward()
    gx, gw = oracle.accumulate_uz_bwd(x, w, gU, gZ, sh)
    assert torch.allclose(x.grad, gx, rtol=1e-12, atol=1e-12)
    assert torch.allclose(w.grad, gw, rtol=1e-12, atol=1e-12)


def test_accumulate_promotes_half_inputs():
    sh = window_shifts(1)
    x = torch.ones(1, 1, 4, 4, dtype=torch.float16)
    w = torch.ones(9, 1, 4, 4, dtype=torch.float16)
    u, z = accumulate_uz_reference(x, w, sh)
    d = normalized_accumulate_uz(x, w, sh)
    assert u.dtype == z.dtype == d.dtype == torch.float32


@pytest.mark.parametrize("log_weights", [False, True])
@pytest.mark.parametrize("table", ["half", "win", "mirror"])
def test_normalized_vs_oracle(log_weights, table):
    sh = {"half": halfplane_shifts(2), "win": window_shifts(2),
          "mirror": explicit_mirror_shifts(halfplane_shifts(2))}[table]
    B, C, H, W = 2, 2, 9, 8
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, C, H, W, dtype=torch.float64, generator=g)
    raw = torch.randn(sh.size(0) * B, C, H, W, dtype=torch.float64, generator=g)
    w = raw * 2 if log_weights else raw.exp()
    w = torch.where(torch.rand(w.shape, generator=g) < 0.1,
                    torch.full_like(w, float("-inf") if log_weights else 0.0), w)
    D, L = normalized_accumulate_uz_reference(x, w, sh, log_weights=log_weights,
                                              return_log_degree=True)
    Do, Lo = oracle.normalized(x, w, sh, log_weights=log_weights, policy="cpu")
    assert torch.allclose(D, Do, rtol=1e-12, atol=1e-12)
    assert torch.allclose(L, Lo, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("log_weights", [False, True])
def test_normalized_gradients_vs_oracle(log_weights):
    sh = halfplane_shifts(2)
    B, C, H, W = 1, 2, 8, 7
    g = torch.Generator().manual_seed(4)
    x = torch.randn(B, C, H, W, dtype=torch.float64, generator=g, requires_grad=True)
    raw = torch.randn(sh.size(0) * B, C, H, W, dtype=torch.float64, generator=g)
    w0 = raw if log_weights else raw.exp()
    mask = torch.rand(w0.shape, generator=g) < 0.1
    w0 = torch.where(mask, torch.full_like(w0, float("-inf") if log_weights else 0.0), w0)
    w = w0.clone().requires_grad_(True)
    D, L = normalized_accumulate_uz(x, w, sh, log_weights=log_weights, return_log_degree=True)
    gD = torch.randn_like(D)
    gL = torch.randn_like(L)
    (D * gD + L * gL).sum().backward()
    gx, gw = oracle.normalized_bwd(x, w0, D.detach(), L.detach(), gD, gL, sh,
                                   log_weights=log_weights)
    assert torch.allclose(x.grad, gx, rtol=1e-10, atol=1e-11)
    # a masked weight gets a zero (not NaN) gradient
    assert torch.isfinite(w.grad).all()
    assert torch.allclose(w.grad, gw, rtol=1e-10, atol=1e-11)


def test_normalized_stable_overflow_closed_form():
    # reference tests/test_normalized_accumulate_uz.py:43-61
    sh = window_shifts(1)
    x = torch.linspace(-1, 1, 20).reshape(1, 1, 5, 4)
    w = torch.full((9, 1, 5, 4), 1.0e38)
    assert torch.isinf(w.view(9, 1, 1, 5, 4).sum(0)).any()
    D, L = normalized_accumulate_uz_reference(x, w, sh, return_log_degree=True)
    exp = torch.stack([roll_gather(x, dx, dy) for dx, dy, _ in sh.tolist()]).mean(0)
    assert torch.isfinite(D).all() and torch.isfinite(L).all()
    torch.testing.assert_close(D, exp, rtol=2e-6, atol=2e-6)


def test_normalized_log_offset_invariance():
    # reference tests/test_normalized_accumulate_uz.py:64-81
    sh = window_shifts(2)
    torch.manual_seed(1)
    x = torch.randn(1, 2, 6, 5)
    logits = 10_000.0 + 3.0 * torch.randn(25, 2, 6, 5)
    d1, l1 = normalized_accumulate_uz_reference(x, logits, sh, log_weights=True,
                                                return_log_degree=True)
    d2, l2 = normalized_accumulate_uz_reference(x, logits + 5_000.0, sh, log_weights=True,
                                                return_log_degree=True)
    assert torch.isfinite(d1).all()
    torch.testing.assert_close(d1, d2, rtol=2e-5, atol=2e-5)
    torch.testing.assert_close(l2 - l1, torch.full_like(l1, 5_000.0), rtol=0, atol=2e-3)


@pytest.mark.parametrize("log_weights", [False, True])
def test_normalized_gradcheck(log_weights):
    # reference tests/test_normalized_accumulate_uz.py:84-99
    torch.manual_seed(2)
    sh = window_shifts(1)
    x = torch.randn(1, 1, 4, 4, dtype=torch.double, requires_grad=True)
    base = torch.randn(9, 1, 4, 4, dtype=torch.double)
    w = (base if log_weights else base.exp()).requires_grad_(True)

    def fn(xx, ww):
        return normalized_accumulate_uz_reference(xx, ww, sh, log_weights=log_weights,
                                                  return_log_degree=True)
    assert torch.autograd.gradcheck(fn, (x, w), eps=1e-6, atol=2e-5)


def test_weight_contract_validation():
    # reference tests/test_normalized_accumulate_uz.py:114-123
    sh = window_shifts(0)
    x = torch.ones(1, 1, 2, 2)
    with pytest.raises(ValueError, match="nonnegative"):
        normalized_accumulate_uz_reference(x, -torch.ones(1, 1, 2, 2), sh)
    with pytest.raises(ValueError, match=r"not NaN or \+inf"):
        normalized_accumulate_uz_reference(x, torch.full((1, 1, 2, 2), torch.inf), sh,
                                           log_weights=True)


def test_type_and_device_errors():
    sh = window_shifts(0)
    with pytest.raises(TypeError):
        accumulate_uz(torch.ones(1, 1, 2, 2, dtype=torch.int32), torch.ones(1, 1, 2, 2), sh)
    with pytest.raises(ValueError):
        accumulate_uz_reference(torch.ones(1, 1, 2, 2), torch.ones(1, 1, 2, 2),
                                torch.zeros(1, 2, dtype=torch.int64))
    with pytest.raises(ValueError):
        shift_gather(torch.ones(1, 1, 2, 2), torch.zeros(1, 4, dtype=torch.int64))


def test_prep_shifts_int64():
    # reference tests/test_index_width.py:9-22
    p = _prep_shifts_for_cuda(torch.tensor([[1, -2, 1]], dtype=torch.int32), torch.device("cpu"))
    assert p.dtype == torch.int64 and p.is_contiguous() and p.tolist() == [[1, -2, 1]]
    big = 2 ** 31 + 17
    p = _prep_shifts_for_cuda(torch.tensor([[big, -big, 0]]), torch.device("cpu"))
    assert p.tolist() == [[big, -big, 0]]


@pytest.mark.parametrize("use_box", [True, False])
def test_metropolis_cpu_paths_vs_oracle(use_box):
    shifts = [(dx, dy, bool(inv)) for dx, dy, inv in halfplane_shifts(2).tolist()]
    B, S, C, H, W = 2, len(shifts), 2, 9, 10
    g = torch.Generator().manual_seed(5)
    wh = torch.nn.functional.softplus(torch.randn(B, S, C, H, W, dtype=torch.float64, generator=g))
    img = torch.randn(B, C, H, W, dtype=torch.float64, generator=g)
    Wo, do = oracle.metropolis(wh, img, halfplane_shifts(2), use_box)
    for fn in (metropolis_aggregate_torch, metropolis_aggregate_fused):
        Wx, dh = fn(wh, img, shifts, use_box, 1e-6)
        assert torch.allclose(Wx, Wo, rtol=1e-12, atol=1e-12)
        assert torch.allclose(dh, do, rtol=1e-12, atol=1e-12)
    wr = wh.clone().requires_grad_(True)
    Wx, dh = metropolis_aggregate(wr, img, shifts, use_box)
    assert torch.allclose(Wx, Wo, rtol=1e-12, atol=1e-12)
    (Wx.sum() + dh.sum()).backward()
    assert torch.isfinite(wr.grad).all()


def test_scalar_reference_vs_oracle():
    sh = window_shifts(2, with_flag=False)
    B, C, H, W = 2, 3, 11, 9
    g = torch.Generator().manual_seed(0)
    x = torch.randn(B, C, H, W, dtype=torch.double, generator=g)
    w = torch.rand(sh.size(0), B, C, dtype=torch.double, generator=g) + 0.1
    U, Z = accumulate_uz_scalar(x, w, sh)
    Uo, Zo = oracle.accumulate_uz_scalar(x, w, sh)
    assert torch.allclose(U, Uo, atol=1e-12) and torch.allclose(Z, Zo, atol=1e-12)
    # (S, B) weights broadcast over channels
    w2 = torch.rand(sh.size(0), B, dtype=torch.double, generator=g)
    U2, _ = accumulate_uz_scalar_reference(x, w2, sh)
    U3, _ = accumulate_uz_scalar_reference(x, w2.unsqueeze(-1).expand(-1, -1, C), sh)
    assert torch.equal(U2, U3)
    with pytest.raises(ValueError):
        accumulate_uz_scalar_reference(x, torch.rand(sh.size(0), B + 1), sh)
