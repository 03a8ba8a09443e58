"""HIP kernels vs the CPU oracle, through the C ABI (via the package ops).

Tolerances (error-bound aware, see helpers.assert_bound): every element of an
accumulation must lie within rtol * (|expected| + sum of |terms|) of the fp64
oracle, rtol = 1e-5 for fp16/bf16/fp32 inputs (fp32 accumulation) and 1e-12
for fp64; half-precision outputs get an extra half-ulp of their own rounding.
Gathers and masks are bit-exact.  Parity cases mirror the reference's own GPU
tests (tests/test_accumulate_uz.py, test_shift_gather.py, test_pair_gather.py,
test_normalized_accumulate_uz.py:126-156) and add fp16/bf16, shifts beyond
the LDS halo, wrapped/huge shift values, explicit-mirror tables and
run-twice determinism.
"""
from __future__ import annotations

import itertools
import sys

import pytest
import torch

import oracle
from helpers import assert_bound, normalized_bwd_cond, out_ulp_for, rtol_for
from neural_shift_cuda import (accumulate_uz, accumulate_uz_reference, accumulate_uz_scalar,
                               metropolis_aggregate, normalized_accumulate_uz, pair_gather,
                               pair_gather_reference, shift_gather, shift_gather_reference)
from neural_shift_cuda_amd.workloads import (box_stack, explicit_mirror_shifts, halfplane_shifts,
                                             window_shifts)

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU"),
]

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _setup():
    oracle.build()
    from neural_shift_cuda_amd import ops
    assert ops._HAS_CUDA_EXT, f"HIP library failed to load: {ops._EXT_IMPORT_ERROR}"


def _case(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _tables():
    return {
        "half1": halfplane_shifts(1),
        "half2": halfplane_shifts(2),
        "half4": halfplane_shifts(4),
        "win2": window_shifts(2),
        "mirror2": explicit_mirror_shifts(halfplane_shifts(2)),
        "far": torch.tensor([[0, 0, 0], [9, 3, 1], [-12, 11, 1], [2, -10, 1], [1000, -7, 1],
                             [-3, 2**31 + 5, 0]]),
    }


def _weights(S, B, C, H, W, sh, dtype, g, masked=True):
    w = torch.randn(S * B, C, H, W, generator=g)
    if masked:
        w = w * box_stack(sh, B, H, W)
    return w.to(dtype)


# ---------------------------------------------------------------------------
# accumulate_uz
# ---------------------------------------------------------------------------

SHAPES = [(1, 3, 16, 16), (2, 3, 31, 29), (3, 6, 33, 47), (2, 2, 40, 64)]


@pytest.mark.parametrize("shape,R", list(itertools.product(SHAPES, [1, 2, 4])))
def test_accumulate_forward_fp32_matches_reference(shape, R):
    # reference tests/test_accumulate_uz.py:48-61 (rtol=atol=1e-5 vs CPU fallback)
    _case(f"accumulate fwd fp32 {shape} R={R}")
    B, C, H, W = shape
    g = torch.Generator().manual_seed(0)
    sh = halfplane_shifts(R)
    x = torch.randn(B, C, H, W, generator=g)
    w = _weights(sh.size(0), B, C, H, W, sh, torch.float32, g)
    U, Z = accumulate_uz(x.to(DEV), w.to(DEV), sh.to(DEV))
    Ur, Zr = accumulate_uz_reference(x, w, sh)
    torch.testing.assert_close(U.cpu(), Ur, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(Z.cpu(), Zr, rtol=1e-5, atol=1e-5)
    Uo, Zo = oracle.accumulate_uz(x, w, sh)
    Us, Zs = oracle.accumulate_uz(x.abs(), w.abs(), sh)
    assert_bound(U, Uo, Us, 1e-5, "U")
    assert_bound(Z, Zo, Zs, 1e-5, "Z")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32, torch.float64])
@pytest.mark.parametrize("table", ["half2", "win2", "mirror2", "far"])
@pytest.mark.parametrize("shape", [(2, 3, 24, 32), (1, 2, 19, 23)])
def test_accumulate_fwd_bwd_vs_oracle(dtype, table, shape):
    _case(f"accumulate fwd+bwd {dtype} {table} {shape}")
    B, C, H, W = shape
    g = torch.Generator().manual_seed(11)
    sh = _tables()[table]
    S = sh.size(0)
    x = torch.randn(B, C, H, W, generator=g).to(dtype)
    w = torch.randn(S * B, C, H, W, generator=g).to(dtype)
    xd = x.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    U, Z = accumulate_uz(xd, wd, sh.to(DEV))
    acc = torch.float64 if dtype == torch.float64 else torch.float32
    assert U.dtype == acc and Z.dtype == acc
    gU = torch.randn(B, C, H, W, generator=g).to(acc)
    gZ = torch.randn(B, C, H, W, generator=g).to(acc)
    (U * gU.to(DEV) + Z * gZ.to(DEV)).sum().backward()
    assert xd.grad.dtype == dtype and wd.grad.dtype == dtype
    rt = rtol_for(dtype)
    Uo, Zo = oracle.accumulate_uz(x, w, sh)
    Us, Zs = oracle.accumulate_uz(x.abs(), w.abs(), sh)
    assert_bound(U, Uo, Us, rt, "U")
    assert_bound(Z, Zo, Zs, rt, "Z")
    gxo, gwo = oracle.accumulate_uz_bwd(x, w, gU, gZ, sh)
    gxs, gws = oracle.accumulate_uz_bwd(x.abs(), w.abs(), gU.abs(), gZ.abs(), sh)
    ou = out_ulp_for(dtype)
    assert_bound(xd.grad, gxo, gxs, rt, "grad_x", ou)
    assert_bound(wd.grad, gwo, gws, rt, "grad_w", ou)


@pytest.mark.parametrize("R", [1, 2])
def test_accumulate_gradcheck(R):
    # reference tests/test_accumulate_uz.py:64-79
    _case(f"accumulate gradcheck R={R}")
    torch.manual_seed(0)
    sh = halfplane_shifts(R).to(DEV)
    B, C, H, W = 1, 2, 6, 5
    x = torch.randn(B, C, H, W, device=DEV, dtype=torch.float64, requires_grad=True)
    w = (torch.randn(sh.size(0) * B, C, H, W, dtype=torch.float64)
         * box_stack(sh.cpu(), B, H, W, torch.float64)).to(DEV).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b: accumulate_uz(a, b, sh), (x, w),
                                    eps=1e-6, atol=1e-5)


def test_accumulate_deterministic():
    _case("accumulate determinism")
    g = torch.Generator().manual_seed(3)
    sh = halfplane_shifts(3).to(DEV)
    x = torch.randn(2, 2, 64, 96, generator=g).to(DEV).requires_grad_(True)
    w = torch.randn(sh.size(0) * 2, 2, 64, 96, generator=g).to(DEV).requires_grad_(True)
    outs = []
    for _ in range(2):
        x.grad = None
        w.grad = None
        U, Z = accumulate_uz(x, w, sh)
        (U.sum() * 0.5 + (Z * Z).sum()).backward()
        outs.append([U.detach().clone(), Z.detach().clone(), x.grad.clone(), w.grad.clone()])
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_accumulate_rejects_bad_arguments():
    x = torch.randn(1, 1, 8, 8, device=DEV)
    w = torch.randn(2, 1, 8, 8, device=DEV)
    with pytest.raises(ValueError):
        accumulate_uz(x, w, torch.zeros(1, 2, dtype=torch.int64, device=DEV))
    with pytest.raises(RuntimeError, match="weights shape"):
        accumulate_uz(x, w, torch.zeros(1, 3, dtype=torch.int64, device=DEV))
    with pytest.raises(RuntimeError, match="1 <= S <= 1024"):
        accumulate_uz(x, torch.randn(1025, 1, 8, 8, device=DEV),
                      torch.zeros(1025, 3, dtype=torch.int64, device=DEV))


# ---------------------------------------------------------------------------
# normalized_accumulate_uz
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.float64])
@pytest.mark.parametrize("log_weights", [False, True])
@pytest.mark.parametrize("table", ["half2", "win2", "far"])
def test_normalized_fwd_bwd_vs_oracle(dtype, log_weights, table):
    _case(f"normalized {dtype} log={log_weights} {table}")
    B, C, H, W = 2, 2, 20, 24
    g = torch.Generator().manual_seed(21)
    sh = _tables()[table]
    S = sh.size(0)
    x = torch.randn(B, C, H, W, generator=g).to(dtype)
    raw = torch.randn(S * B, C, H, W, generator=g)
    w = (2 * raw) if log_weights else raw.exp()
    pick = torch.rand(w.shape, generator=g)
    w = torch.where(pick < 0.1, torch.full_like(w, float("-inf") if log_weights else 0.0), w)
    if log_weights:
        w = torch.where(pick > 0.99, 80.0 * torch.sign(raw), w)  # +-80 outliers
    w[:, 0, 3, 4] = float("-inf") if log_weights else 0.0      # an empty row
    w = w.to(dtype)
    xd = x.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    D, L = normalized_accumulate_uz(xd, wd, sh.to(DEV), log_weights=log_weights,
                                    return_log_degree=True)
    gD = torch.randn(B, C, H, W, generator=g).to(D.dtype)
    gL = torch.randn(B, C, H, W, generator=g).to(D.dtype)
    (D * gD.to(DEV) + L * gL.to(DEV)).sum().backward()
    rt = rtol_for(dtype)
    Do, Lo = oracle.normalized(x, w, sh, log_weights=log_weights, policy="gpu")
    Ds, _ = oracle.normalized(x.abs(), w, sh, log_weights=log_weights, policy="gpu")
    assert_bound(D, Do, Ds, rt, "D")
    assert_bound(L, Lo, Lo.abs().nan_to_num(posinf=0, neginf=0) + 1.0, rt, "log_C")
    gxo, gwo = oracle.normalized_bwd(x, w, Do, Lo, gD, gL, sh, log_weights=log_weights)
    # x[p+s] - D enters each weight gradient: D's own error (<= rtol * Ds) propagates,
    # so the scale takes Ds = sum w|x| / C >= |D| in D's place
    gxs, gws = oracle.normalized_bwd(x.abs(), w, -Ds, Lo, gD.abs(), gL.abs(), sh,
                                     log_weights=log_weights)
    ou = out_ulp_for(dtype)
    # exp(l - L) in the gradient carries the forward's L error and |l - L|
    # relative rounding per term: derived per element
    gxc, gwc = normalized_bwd_cond(x, w, Lo, gD, gL, Ds, sh, log_weights=log_weights,
                                   acc_dtype=dtype)
    assert_bound(xd.grad, gxo, gxs, rt, "grad_x", ou, extra=gxc)
    assert_bound(wd.grad, gwo, gws, rt, "grad_w", ou, extra=gwc)


@pytest.mark.parametrize("log_weights", [False, True])
def test_normalized_matches_reference_test_cuda_case(log_weights):
    # reference tests/test_normalized_accumulate_uz.py:126-156 (fp64, 1e-10 / 1e-9)
    torch.manual_seed(3)
    sh = window_shifts(2)
    B, C, H, W = 1, 2, 8, 7
    x0 = torch.randn(B, C, H, W, dtype=torch.double)
    raw = torch.randn(sh.size(0) * B, C, H, W, dtype=torch.double)
    w0 = raw if log_weights else raw.exp()
    xc = x0.to(DEV).requires_grad_(True)
    wc = w0.to(DEV).requires_grad_(True)
    xr = x0.clone().requires_grad_(True)
    wr = w0.clone().requires_grad_(True)
    from neural_shift_cuda import normalized_accumulate_uz_reference as ref
    dc, lc = normalized_accumulate_uz(xc, wc, sh.to(DEV), log_weights=log_weights,
                                      return_log_degree=True)
    dr, lr = ref(xr, wr, sh, log_weights=log_weights, return_log_degree=True)
    torch.testing.assert_close(dc.cpu(), dr, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(lc.cpu(), lr, rtol=1e-10, atol=1e-10)
    gd = torch.randn_like(dc)
    gl = torch.randn_like(lc)
    (dc * gd + lc * gl).sum().backward()
    (dr * gd.cpu() + lr * gl.cpu()).sum().backward()
    torch.testing.assert_close(xc.grad.cpu(), xr.grad, rtol=1e-9, atol=1e-9)
    torch.testing.assert_close(wc.grad.cpu(), wr.grad, rtol=1e-9, atol=1e-9)


def test_normalized_nan_policy_and_overflow():
    sh = window_shifts(1)
    x = torch.linspace(-1, 1, 20).reshape(1, 1, 5, 4)
    w = torch.full((9, 1, 5, 4), 1.0e38)
    D, L = normalized_accumulate_uz(x.to(DEV), w.to(DEV), sh.to(DEV), return_log_degree=True)
    Do, Lo = oracle.normalized(x, w, sh, log_weights=False, policy="gpu")
    assert torch.isfinite(D).all() and torch.isfinite(L).all()
    torch.testing.assert_close(D.cpu(), Do.float(), rtol=2e-6, atol=2e-6)
    torch.testing.assert_close(L.cpu(), Lo.float(), rtol=1e-6, atol=1e-5)
    w2 = torch.rand(9, 1, 5, 4) + 0.1
    w2[4, 0, 2, 2] = -1.0
    D2, L2 = normalized_accumulate_uz(x.to(DEV), w2.to(DEV), sh.to(DEV), validate=False,
                                      return_log_degree=True)
    assert torch.isnan(D2[0, 0, 2, 2]) and torch.isnan(L2[0, 0, 2, 2])
    assert int(torch.isfinite(D2).sum()) == 19


# ---------------------------------------------------------------------------
# gathers
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32, torch.float64])
@pytest.mark.parametrize("shape,R", list(itertools.product(
    [(1, 8, 16, 16), (2, 16, 31, 29), (4, 3, 64, 64)], [0, 1, 2, 5])))
def test_gathers_bit_exact(dtype, shape, R):
    # reference tests/test_shift_gather.py:35-81, test_pair_gather.py:38-57
    _case(f"gathers {dtype} {shape} R={R}")
    B, C, H, W = shape
    g = torch.Generator().manual_seed(0)
    guide = torch.randn(B, C, H, W, generator=g).to(dtype)
    sh = halfplane_shifts(R)
    gs, m = shift_gather(guide.to(DEV), sh.to(DEV))
    go, mo = oracle.shift_gather(guide, sh)
    assert gs.dtype == dtype and m.dtype == dtype
    assert torch.equal(gs.cpu(), go) and torch.equal(m.cpu(), mo)
    p, pm = pair_gather(guide.to(DEV), sh.to(DEV))
    po, pmo = oracle.pair_gather(guide, sh)
    assert torch.equal(p.cpu(), po) and torch.equal(pm.cpu(), pmo)
    if dtype in (torch.float32, torch.float64):
        gr, mr = shift_gather_reference(guide, sh)
        assert torch.equal(gs.cpu(), gr) and torch.equal(m.cpu(), mr)
        pr, _ = pair_gather_reference(guide, sh)
        assert torch.equal(p.cpu(), pr)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.bfloat16])
@pytest.mark.parametrize("pair", [False, True])
def test_gather_backward_vs_oracle(dtype, pair):
    _case(f"gather backward {dtype} pair={pair}")
    B, C, H, W = 2, 4, 13, 16
    g = torch.Generator().manual_seed(7)
    sh = _tables()["far"][:, :2].contiguous()
    guide = torch.randn(B, C, H, W, generator=g).to(dtype).to(DEV).requires_grad_(True)
    fn = pair_gather if pair else shift_gather
    out, _ = fn(guide, sh.to(DEV))
    gout = torch.randn(out.shape, generator=g).to(dtype)
    out.backward(gout.to(DEV))
    ref = (oracle.pair_gather_bwd if pair else oracle.shift_gather_bwd)(gout, sh, B, C, H, W)
    scale = (oracle.pair_gather_bwd if pair else oracle.shift_gather_bwd)(gout.abs(), sh, B, C, H, W)
    assert_bound(guide.grad, ref, scale, rtol_for(dtype), "grad_guide", out_ulp_for(dtype))
    g1 = guide.grad.clone()
    guide.grad = None
    out, _ = fn(guide, sh.to(DEV))
    out.backward(gout.to(DEV))
    assert torch.equal(g1, guide.grad)  # deterministic, atomic-free


def test_gather_gradcheck():
    # reference tests/test_shift_gather.py:88-101, test_pair_gather.py:64-76
    sh = halfplane_shifts(2).to(DEV)
    guide = torch.randn(1, 2, 5, 5, device=DEV, dtype=torch.float64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda t: shift_gather(t, sh)[0], (guide,), eps=1e-6, atol=1e-5)
    assert torch.autograd.gradcheck(lambda t: pair_gather(t, sh)[0], (guide,), eps=1e-6, atol=1e-5)


# ---------------------------------------------------------------------------
# Metropolis
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.float64])
@pytest.mark.parametrize("use_box", [True, False])
@pytest.mark.parametrize("shape", [(2, 2, 24, 32), (1, 1, 19, 21)])
def test_metropolis_vs_oracle(dtype, use_box, shape):
    _case(f"metropolis {dtype} box={use_box} {shape}")
    B, C, H, W = shape
    sh = halfplane_shifts(3)
    shifts = [(dx, dy, bool(inv)) for dx, dy, inv in sh.tolist()]
    S = sh.size(0)
    g = torch.Generator().manual_seed(5)
    wh = torch.nn.functional.softplus(torch.randn(B, S, C, H, W, generator=g)).to(dtype)
    img = torch.randn(B, C, H, W, generator=g).to(dtype)
    with torch.no_grad():
        Wx, dh = metropolis_aggregate(wh.to(DEV), img.to(DEV), shifts, use_box)
    assert Wx.dtype == dtype and dh.dtype == dtype
    Wo, do = oracle.metropolis(wh, img, sh, use_box)
    # Wx = x - d_hat x + K_hat x: bound by |x|(1 + d_hat) + K_hat|x|
    Ws, _ = oracle.metropolis(wh, img.abs(), sh, use_box)
    scale = Ws.abs() + 2 * img.double().abs() * (1 + do.abs())
    rt = rtol_for(dtype)
    ou = out_ulp_for(dtype)
    assert_bound(Wx, Wo, scale, rt, "Wx", ou)
    assert_bound(dh, do, do.abs(), rt, "d_hat", ou)


def test_metropolis_training_path_gradients():
    sh = halfplane_shifts(2)
    shifts = [(dx, dy, bool(inv)) for dx, dy, inv in sh.tolist()]
    B, S, C, H, W = 1, sh.size(0), 2, 16, 20
    g = torch.Generator().manual_seed(6)
    wh = torch.nn.functional.softplus(torch.randn(B, S, C, H, W, dtype=torch.float64, generator=g))
    img = torch.randn(B, C, H, W, dtype=torch.float64, generator=g)
    wg = wh.to(DEV).requires_grad_(True)
    Wx, dh = metropolis_aggregate(wg, img.to(DEV), shifts, True)
    Wo, do = oracle.metropolis(wh, img, sh, True)
    assert torch.allclose(Wx.detach().cpu(), Wo, rtol=1e-12, atol=1e-12)
    (Wx.sum() + dh.square().sum()).backward()
    wc = wh.clone().requires_grad_(True)
    from neural_shift_cuda.metropolis import metropolis_aggregate_fused
    Wr, dr = metropolis_aggregate_fused(wc, img, shifts, True)
    (Wr.sum() + dr.square().sum()).backward()
    torch.testing.assert_close(wg.grad.cpu(), wc.grad, rtol=1e-10, atol=1e-10)


def test_metropolis_exact_symmetry():
    sh = halfplane_shifts(2)
    shifts = [(dx, dy, bool(inv)) for dx, dy, inv in sh.tolist()]
    B, S, C, H, W = 1, sh.size(0), 1, 32, 48
    g = torch.Generator().manual_seed(9)
    wh = torch.nn.functional.softplus(torch.randn(B, S, C, H, W, generator=g)).to(DEV)
    pairs = [((1, 2), (2, 3)), ((0, 0), (1, 47)), ((10, 10), (12, 11)), ((31, 47), (31, 46))]
    with torch.no_grad():
        for use_box in (True, False):
            for i, j in pairs:
                ei = torch.zeros(B, C, H, W, device=DEV)
                ej = torch.zeros(B, C, H, W, device=DEV)
                ei[0, 0, i[0], i[1]] = 1
                ej[0, 0, j[0], j[1]] = 1
                Wej, _ = metropolis_aggregate(wh, ej, shifts, use_box)
                Wei, _ = metropolis_aggregate(wh, ei, shifts, use_box)
                assert Wej[0, 0, i[0], i[1]].item() == Wei[0, 0, j[0], j[1]].item()


# ---------------------------------------------------------------------------
# accumulate_uz_scalar
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dtype", [torch.float32, torch.float64, torch.bfloat16])
@pytest.mark.parametrize("shape", [(2, 3, 11, 9), (2, 3, 64, 96), (1, 2, 100, 200)])
@pytest.mark.parametrize("table", ["win2", "far"])
def test_scalar_vs_oracle(dtype, shape, table):
    # tiles of 64 x 32 pixels: one partial tile, 2 x 2 tiles, 4 x 4 with partial
    # edges; "far" has shifts beyond the 8-pixel LDS halo (read from HBM)
    _case(f"scalar {dtype} {shape} {table}")
    B, C, H, W = shape
    sh = window_shifts(2, with_flag=False) if table == "win2" else \
        _tables()["far"][:, :2].contiguous()
    S = sh.size(0)
    g = torch.Generator().manual_seed(12)
    x = torch.randn(B, C, H, W, generator=g).to(dtype)
    w = (torch.rand(S, B, C, generator=g) + 0.1).to(dtype)
    xd = x.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    U, Z = accumulate_uz_scalar(xd, wd, sh.to(DEV))
    gU = torch.randn(B, C, H, W, generator=g).to(U.dtype)
    gZ = torch.randn(B, C, H, W, generator=g).to(U.dtype)
    (U * gU.to(DEV) + Z * gZ.to(DEV)).sum().backward()
    rt = rtol_for(dtype)
    Uo, Zo = oracle.accumulate_uz_scalar(x, w, sh)
    Us, Zs = oracle.accumulate_uz_scalar(x.abs(), w.abs(), sh)
    assert_bound(U, Uo, Us, rt, "U")
    assert_bound(Z, Zo, Zs, rt, "Z")
    gxo, gwo = oracle.accumulate_uz_scalar_bwd(x, w, gU, gZ, sh)
    gxs, gws = oracle.accumulate_uz_scalar_bwd(x.abs(), w.abs(), gU.abs(), gZ.abs(), sh)
    assert_bound(xd.grad, gxo, gxs, rt, "grad_x", out_ulp_for(dtype))
    assert_bound(wd.grad, gwo, gws, rt, "grad_w", out_ulp_for(dtype))
