"""Circular mirrors (``periodic_inverse=True``; row code 2 under NSH_SHIFT_CODES).

The periodic symmetric operator of a half-plane table equals the reference's
own construction with explicit rows (nekde_drunet_attn_patch.py:350-366):
every row forward-only, each has_inverse row followed by (-dx, -dy) with the
weight rolled by (dx, dy).  That identity pins the circular mirror: the CPU
paths and the HIP kernels (scatter, far-row and gather forms) are compared
with the C oracle run on the explicit table, gradients folded back onto the
half-plane weights (grad w_s = g_fwd + roll(g_mirror, -s)).  Tolerances: the
error-bound rule of the other accumulation tests (rtol 1e-5 fp32-class,
1e-12 fp64; the normalized gradients add the derived conditioning term of
helpers.normalized_bwd_cond; output rounding for fp16).
"""
from __future__ import annotations

import sys

import pytest
import torch

import oracle
from helpers import assert_bound, normalized_bwd_cond, out_ulp_for, rtol_for
from neural_shift_cuda import accumulate_uz, normalized_accumulate_uz
from neural_shift_cuda_amd import _C
from neural_shift_cuda_amd.workloads import halfplane_shifts

HAS_GPU = torch.cuda.is_available()
DEV = torch.device("cuda:0")
_CODE = {torch.float16: 1, torch.bfloat16: 2, torch.float32: 3, torch.float64: 4}


def _case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _setup():
    oracle.build()


def _table(name):
    return {
        "half1": halfplane_shifts(1),
        "half2": halfplane_shifts(2),
        "half6": halfplane_shifts(6),
        "half8": halfplane_shifts(8),
        "far": torch.tensor([[0, 0, 0], [9, 3, 1], [-2, 1, 1], [1, -10, 1], [3, 2, 0]]),
        "selfinv": torch.tensor([[0, 0, 1], [1, 0, 1], [0, 1, 1], [-1, 2, 0]]),
    }[name]


def _explicit(sh: torch.Tensor, w: torch.Tensor, B: int):
    """(explicit table, explicit weights, row index of each mirror or -1)."""
    S = sh.size(0)
    wv = w.view(S, B, *w.shape[1:])
    rows, planes, mirror = [], [], []
    for s, (dx, dy, inv) in enumerate(sh.tolist()):
        rows.append((dx, dy, 0))
        planes.append(wv[s])
        if inv:
            mirror.append(len(rows))
            rows.append((-dx, -dy, 0))
            planes.append(torch.roll(wv[s], shifts=(dx, dy), dims=(-2, -1)))
        else:
            mirror.append(-1)
    pos = []
    r = 0
    for s in range(S):
        pos.append(r)
        r += 2 if mirror[s] >= 0 else 1
    return (torch.tensor(rows, dtype=torch.int64), torch.stack(planes).reshape(-1, *w.shape[1:]),
            pos, mirror)


def _fold(g_exp: torch.Tensor, sh: torch.Tensor, pos, mirror, B: int) -> torch.Tensor:
    """Gradient of the explicit rows folded back onto the half-plane."""
    gv = g_exp.view(-1, B, *g_exp.shape[1:])
    out = []
    for s, (dx, dy, inv) in enumerate(sh.tolist()):
        g = gv[pos[s]]
        if mirror[s] >= 0:
            g = g + torch.roll(gv[mirror[s]], shifts=(-dx, -dy), dims=(-2, -1))
        out.append(g)
    return torch.stack(out).reshape(-1, *g_exp.shape[1:])


def _inputs(B, C, H, W, S, dtype, seed, log_weights=None):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, C, H, W, generator=g).to(dtype)
    if log_weights is None:      # signed weights for the plain accumulation
        w = torch.randn(S * B, C, H, W, generator=g)
    elif log_weights:
        w = 2 * torch.randn(S * B, C, H, W, generator=g)
    else:
        w = torch.nn.functional.softplus(torch.randn(S * B, C, H, W, generator=g))
    acc = torch.float64 if dtype == torch.float64 else torch.float32
    g1 = torch.randn(B, C, H, W, generator=g).to(acc)
    g2 = torch.randn(B, C, H, W, generator=g).to(acc)
    return x, w.to(dtype), g1, g2


# ---------------------------------------------------------------------------
# CPU: the package's CPU paths against the explicit construction
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("table", ["half2", "far", "selfinv"])
def test_cpu_periodic_matches_explicit_rows(table):
    sh = _table(table)
    B, C, H, W = 2, 2, 11, 13
    x, w, gU, gZ = _inputs(B, C, H, W, sh.size(0), torch.float64, 3)
    xr, wr = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    U, Z = accumulate_uz(xr, wr, sh, periodic_inverse=True)
    torch.autograd.backward([U, Z], [gU, gZ])
    xe, we = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    te, wexp, pos, mirror = _explicit(sh, we, B)
    Ue, Ze = accumulate_uz(xe, wexp, te)
    torch.autograd.backward([Ue, Ze], [gU, gZ])
    torch.testing.assert_close(U, Ue, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(Z, Ze, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(xr.grad, xe.grad, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(wr.grad, we.grad, rtol=1e-12, atol=1e-12)
    # the normalized op
    for log_weights in (False, True):
        _, wn, _, _ = _inputs(B, C, H, W, sh.size(0), torch.float64, 4, log_weights)
        D, L = normalized_accumulate_uz(x, wn, sh, log_weights=log_weights,
                                        return_log_degree=True, periodic_inverse=True)
        te, wnexp, _, _ = _explicit(sh, wn, B)
        De, Le = normalized_accumulate_uz(x, wnexp, te, log_weights=log_weights,
                                          return_log_degree=True)
        torch.testing.assert_close(D, De, rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(L, Le, rtol=1e-12, atol=1e-12)
    # periodic differs from the finite-window operator near the border
    Ub, _ = accumulate_uz(x, w, sh)
    assert not torch.allclose(Ub, U.detach())


# ---------------------------------------------------------------------------
# GPU: every kernel form against the oracle on the explicit table
# ---------------------------------------------------------------------------

ACC_SHAPES = [
    (torch.float32, (1, 2, 1033, 1036)),   # scatter path, partial edge tiles
    (torch.float64, (1, 1, 1033, 1034)),   # scatter path, fp64 tiles
    (torch.float16, (2, 1, 136, 216)),     # scatter path, 16-bit (fp32 gx partials)
    (torch.float32, (64, 1, 40, 200)),     # scatter path, 2 x 2 tiles: the window wraps onto the other tile
    (torch.float32, (1, 1, 40, 52)),       # gather kernels (too small to scatter)
]


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
@pytest.mark.parametrize("dtype,shape", ACC_SHAPES)
@pytest.mark.parametrize("table", ["half2", "half6", "far", "selfinv"])
def test_gpu_accumulate_periodic_vs_oracle(dtype, shape, table):
    _case(f"accumulate periodic {dtype} {shape} {table}")
    sh = _table(table)
    B, C, H, W = shape
    S = sh.size(0)
    x, w, gU, gZ = _inputs(B, C, H, W, S, dtype, 21)
    xd = x.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    U, Z = accumulate_uz(xd, wd, sh.to(DEV), periodic_inverse=True)
    torch.autograd.backward([U, Z], [gU.to(DEV), gZ.to(DEV)])
    torch.cuda.synchronize()
    te, we, pos, mirror = _explicit(sh, w, B)
    rt = rtol_for(dtype)
    Uo, Zo = oracle.accumulate_uz(x, we, te)
    Us, Zs = oracle.accumulate_uz(x.abs(), we.abs(), te)
    assert_bound(U, Uo, Us, rt, "U")
    assert_bound(Z, Zo, Zs, rt, "Z")
    del Uo, Zo, Us, Zs
    gxo, gwo = oracle.accumulate_uz_bwd(x, we, gU, gZ, te)
    gxs, gws = oracle.accumulate_uz_bwd(x.abs(), we.abs(), gU.abs(), gZ.abs(), te)
    ou = out_ulp_for(dtype)
    assert_bound(xd.grad, gxo, gxs, rt, "grad_x", ou)
    assert_bound(wd.grad, _fold(gwo, sh, pos, mirror, B), _fold(gws, sh, pos, mirror, B), rt,
                 "grad_w", ou)


NORM_SHAPES = [
    (torch.float32, (1, 2, 72, 200)),      # scatter path
    (torch.float64, (1, 1, 104, 104)),     # scatter path, fp64
    (torch.float32, (1, 1, 30, 44)),       # gather kernels
]


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
@pytest.mark.parametrize("dtype,shape", NORM_SHAPES)
@pytest.mark.parametrize("table", ["half1", "half6", "far", "selfinv"])
@pytest.mark.parametrize("log_weights", [False, True])
def test_gpu_normalized_periodic_vs_oracle(dtype, shape, table, log_weights):
    _case(f"normalized periodic {dtype} {shape} {table} log={log_weights}")
    sh = _table(table)
    B, C, H, W = shape
    S = sh.size(0)
    x, w, gD, gL = _inputs(B, C, H, W, S, dtype, 22, log_weights)
    xd = x.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    D, L = normalized_accumulate_uz(xd, wd, sh.to(DEV), log_weights=log_weights,
                                    return_log_degree=True, validate=False,
                                    periodic_inverse=True)
    torch.autograd.backward([D, L], [gD.to(D.dtype).to(DEV), gL.to(D.dtype).to(DEV)])
    torch.cuda.synchronize()
    te, we, pos, mirror = _explicit(sh, w, B)
    rt = rtol_for(dtype)
    Do, Lo = oracle.normalized(x, we, te, log_weights=log_weights, policy="gpu")
    Ds, _ = oracle.normalized(x.abs(), we, te, log_weights=log_weights, policy="gpu")
    assert_bound(D, Do, Ds, rt, "D")
    assert_bound(L, Lo, Lo.abs().nan_to_num(posinf=0, neginf=0) + 1.0, rt, "log_C")
    gxo, gwo = oracle.normalized_bwd(x, we, Do, Lo, gD, gL, te, log_weights=log_weights)
    gxs, gws = oracle.normalized_bwd(x.abs(), we, -Ds, Lo, gD.abs(), gL.abs(), te,
                                     log_weights=log_weights)
    ou = out_ulp_for(dtype)
    gxc, gwc = normalized_bwd_cond(x, we, Lo, gD, gL, Ds, te, log_weights=log_weights,
                                   acc_dtype=dtype)
    assert_bound(xd.grad, gxo, gxs, rt, "grad_x", ou, extra=gxc)
    assert_bound(wd.grad, _fold(gwo, sh, pos, mirror, B), _fold(gws, sh, pos, mirror, B),
                 rt, "grad_w", ou, extra=_fold(gwc, sh, pos, mirror, B))


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
def test_gpu_periodic_scatter_eligibility_and_determinism():
    """The circular mirror keeps the scatter path (workspace in use) and is
    bitwise reproducible."""
    _case("periodic scatter determinism")
    sh = _table("half6")
    B, C, H, W = 1, 2, 1033, 1036
    assert int(_C._lib.nsh_accumulate_uz_workspace_bytes(sh.size(0), B, C, H, W, 3, 0)) > 0
    x, w, _, _ = _inputs(B, C, H, W, sh.size(0), torch.float32, 23)
    xd, wd, shd = x.to(DEV), w.to(DEV), sh.to(DEV)
    a = accumulate_uz(xd, wd, shd, periodic_inverse=True)
    b = accumulate_uz(xd, wd, shd, periodic_inverse=True)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


# ---------------------------------------------------------------------------
# The table's third column is the reference's flag unless an extension is
# asked for: any nonzero has_inverse is the reference's mirror (dropped
# where its source wraps), on the CPU fallback and through the C ABI
# ---------------------------------------------------------------------------

def _flag_variants(sh):
    """The same table with every nonzero has_inverse replaced by 2, 4, 7, -1."""
    out = []
    for v in (2, 4, 7, -1):
        t = sh.clone()
        t[:, 2] = torch.where(t[:, 2] != 0, torch.full_like(t[:, 2], v), t[:, 2])
        out.append(t)
    return out


@pytest.mark.parametrize("table", ["half2", "far", "selfinv"])
def test_cpu_nonzero_has_inverse_is_reference_mirror(table):
    sh = _table(table)
    B, C, H, W = 1, 2, 11, 13
    x, w, _, _ = _inputs(B, C, H, W, sh.size(0), torch.float64, 5, log_weights=False)
    U, Z = accumulate_uz(x, w, sh)
    Uo, Zo = oracle.accumulate_uz(x, w, sh)
    torch.testing.assert_close(U, Uo, rtol=1e-12, atol=1e-12)
    D = normalized_accumulate_uz(x, w, sh)
    for t in _flag_variants(sh):
        U2, Z2 = accumulate_uz(x, w, t)
        assert torch.equal(U2, U) and torch.equal(Z2, Z), t[:, 2].tolist()
        assert torch.equal(normalized_accumulate_uz(x, w, t), D)


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
@pytest.mark.parametrize("shape", [(1, 2, 72, 200), (1, 1, 30, 44)])
def test_gpu_nonzero_has_inverse_is_reference_mirror(shape):
    """Reference tables with has_inverse values other than 0/1 (including
    the values the row codes use) give the reference's masked mirror."""
    _case(f"has_inverse values {shape}")
    sh = _table("half6")
    B, C, H, W = shape
    x, w, gU, gZ = _inputs(B, C, H, W, sh.size(0), torch.float32, 6, log_weights=False)
    xd, wd = x.to(DEV), w.to(DEV)
    U, Z = accumulate_uz(xd, wd, sh.to(DEV))
    D, L = normalized_accumulate_uz(xd, wd, sh.to(DEV), return_log_degree=True)
    Uo, Zo = oracle.accumulate_uz(x, w, sh)
    Us, Zs = oracle.accumulate_uz(x.abs(), w.abs(), sh)
    assert_bound(U, Uo, Us, 1e-5, "U")
    for t in _flag_variants(sh):
        U2, Z2 = accumulate_uz(xd, wd, t.to(DEV))
        D2, L2 = normalized_accumulate_uz(xd, wd, t.to(DEV), return_log_degree=True)
        assert torch.equal(U2, U) and torch.equal(Z2, Z), t[:, 2].tolist()
        assert torch.equal(D2, D) and torch.equal(L2, L), t[:, 2].tolist()
