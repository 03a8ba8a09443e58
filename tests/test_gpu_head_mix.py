"""normalized_accumulate_uz of head-mixed weights with the mixing product in
the forward kernel's weight load (nsh_normalized_accumulate_uz_forward_mixed,
ops.normalized_accumulate_uz_mixed): channel c of shift s and batch b weighs
sum_j mix[c, j] * w[s*B+b, j], which the attention installers otherwise form
as a (S, B, C, H, W) stack before the accumulation (reference
nekde_drunet_attn_patch.py:117-140, then :368-370).

Checks, on shapes the scatter path serves (partial edge tiles, several
planes, 2..4 heads, every dtype):
* against the fp64 oracle run on the heads mixed in fp64 from the kernel's
  own rounded inputs (head weights in their dtype, the mix in the
  accumulator type);
* against the library's unfused path (heads mixed by a matmul, then the
  plain op) within the sum of both bounds;
* tables with mirror rows, rows beyond the 8-pixel halo (the gather form
  inside the kernel, which mixes its weight reads too), the forward box and
  circular mirrors (row codes), masked pixels and a fully masked row;
* head counts and shapes the entry point does not serve (NSH_ERR_UNSUPPORTED,
  the op mixing first), the autograd route (mixing first, gradients to the
  heads and the matrix), and the NeKDe / GASD installers without autograd
  against their autograd route.

Tolerance: the rule of tests/helpers.py (rtol 1e-5 of the term scale for
fp32-accumulated inputs, 1e-12 for fp64).  Mixing at most 4 positive terms
in the accumulator type perturbs each weight by at most 4u relatively, which
moves D by at most 4u (|D| + sum a|x| / sum a): inside the bound.
"""
from __future__ import annotations

import sys

import pytest
import torch

import oracle
from helpers import assert_bound, rtol_for
from neural_shift_cuda_amd import _C
from neural_shift_cuda_amd.ops import normalized_accumulate_uz, normalized_accumulate_uz_mixed
from neural_shift_cuda_amd.workloads import box_stack, explicit_mirror_shifts, halfplane_shifts

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


def _table(name):
    return {
        "half6": halfplane_shifts(6),
        "mirror3": explicit_mirror_shifts(halfplane_shifts(3)),
        "far": torch.tensor([[0, 1, 1], [9, 3, 1], [-2, 1, 1], [1, -10, 1], [3, 2, 0],
                             [2, 2, 1], [-12, 0, 0]]),
    }[name]


def _inputs(dtype, shape, S, heads, seed):
    """x, positive head weights with masked pixels (every head 0) and one
    fully masked row, and a softmax mixing matrix."""
    B, C, H, W = shape
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, C, H, W, generator=g).to(dtype)
    hw = torch.randn(S * B, heads, H, W, generator=g).exp()
    hw = hw * (torch.rand(S * B, 1, H, W, generator=g) >= 0.1)   # masked pixels
    hw[:, :, 3, 4] = 0.0                                        # an empty row
    mix = torch.softmax(torch.randn(C, heads, generator=g, dtype=torch.float64), dim=1)
    return x, hw.to(dtype), mix


def _oracle_weights(hw, mix, C, acc):
    """The heads mixed in fp64 from the kernel's inputs: head weights as
    stored, the matrix rounded to the accumulator type."""
    SB, h, H, W = hw.shape
    m = mix.to(acc).double()
    return torch.matmul(m, hw.double().reshape(SB, h, H * W)).view(SB, C, H, W)


def _oracle_operands(sh, w, B, H, W, periodic, box):
    """(table, weights) of the same operator without row codes: the forward
    box as masked weights, circular mirrors as explicit rows (-dx, -dy) whose
    planes are the forward planes rolled by (dx, dy)."""
    if box:
        return sh, w * box_stack(sh, B, H, W, dtype=w.dtype)
    if not periodic:
        return sh, w
    S = sh.size(0)
    wv = w.view(S, B, *w.shape[1:])
    rows, planes = [], []
    for s, (dx, dy, inv) in enumerate(sh.tolist()):
        rows.append((dx, dy, 0))
        planes.append(wv[s])
        if inv:
            rows.append((-dx, -dy, 0))
            planes.append(torch.roll(wv[s], shifts=(dx, dy), dims=(-2, -1)))
    return torch.tensor(rows, dtype=torch.int64), torch.stack(planes).reshape(-1, *w.shape[1:])


CASES = [
    (torch.float32, (1, 3, 72, 200), 2),
    (torch.float32, (2, 2, 104, 138), 4),
    (torch.float16, (2, 3, 104, 136), 3),
    (torch.bfloat16, (1, 2, 80, 140), 4),
    (torch.float64, (1, 3, 72, 76), 2),
]


@pytest.mark.parametrize("dtype,shape,heads", CASES)
@pytest.mark.parametrize("table", ["half6", "mirror3", "far"])
@pytest.mark.parametrize("mode", ["reference", "box", "periodic"])
def test_mixed_forward_vs_oracle_and_unfused(dtype, shape, heads, table, mode):
    B, C, H, W = shape
    sh = _table(table)
    S = sh.size(0)
    periodic, box = mode == "periodic", mode == "box"
    _case(f"head mix {dtype} {shape} heads={heads} {table} {mode}")
    x, hw, mix = _inputs(dtype, shape, S, heads, 71)
    acc = torch.float64 if dtype == torch.float64 else torch.float32
    xd, hwd = x.to(DEV), hw.to(DEV)
    # the entry point serves this case itself (no fallback)
    table_d, codes = (sh.to(DEV), False)
    if periodic or box:
        from neural_shift_cuda_amd.ops import _mirror_table
        table_d, codes = _mirror_table(sh.to(DEV), periodic, box)
    out = _C.normalized_accumulate_uz_forward_mixed(xd, hwd, mix, table_d, row_codes=codes)
    assert out is not None, "the scatter path should serve this shape"
    with torch.no_grad():
        D, L = normalized_accumulate_uz_mixed(xd, hwd, mix.to(DEV), sh.to(DEV),
                                              return_log_degree=True, periodic_inverse=periodic,
                                              box_forward=box)
    torch.cuda.synchronize()
    assert torch.equal(D, out[0]) and torch.equal(L, out[1])
    rt = rtol_for(dtype)
    to, wo = _oracle_operands(sh, _oracle_weights(hw, mix, C, acc), B, H, W, periodic, box)
    Do, Lo = oracle.normalized(x, wo, to, log_weights=False, policy="gpu")
    Ds, _ = oracle.normalized(x.abs(), wo, to, log_weights=False, policy="gpu")
    assert_bound(D, Do, Ds, rt, "D")
    assert_bound(L, Lo, Lo.abs().nan_to_num(posinf=0, neginf=0) + 1.0, rt, "log_C")
    # the unfused path: heads mixed by a matmul in the accumulator type
    mixed = torch.matmul(mix.to(device=DEV, dtype=acc),
                         hwd.to(acc).reshape(S * B, heads, H * W)).view(S * B, C, H, W)
    Du, Lu = normalized_accumulate_uz(xd.to(acc), mixed, sh.to(DEV), return_log_degree=True,
                                      validate=False, periodic_inverse=periodic,
                                      box_forward=box)
    assert_bound(D, Du.double().cpu(), Ds, 2 * rt, "D vs unfused")
    assert_bound(L, Lu.double().cpu(), Lo.abs().nan_to_num(posinf=0, neginf=0) + 1.0, 2 * rt,
                 "log_C vs unfused")


def test_mixed_forward_deterministic():
    _case("head mix determinism")
    sh = _table("half6")
    x, hw, mix = _inputs(torch.float32, (1, 3, 72, 200), sh.size(0), 3, 5)
    runs = []
    for _ in range(2):
        with torch.no_grad():
            runs.append(normalized_accumulate_uz_mixed(x.to(DEV), hw.to(DEV), mix.to(DEV),
                                                       sh.to(DEV), return_log_degree=True))
    for a, b in zip(*runs):
        assert torch.equal(a.nan_to_num(), b.nan_to_num())


@pytest.mark.parametrize("shape,heads,why", [((1, 3, 16, 20), 2, "shape"),
                                             ((1, 3, 72, 200), 5, "heads"),
                                             ((1, 2, 72, 200), 1, "heads")])
def test_mixed_forward_unsupported_falls_back(shape, heads, why):
    """The entry point reports NSH_ERR_UNSUPPORTED (None from _C) and the op
    mixes first: the results still meet the oracle's bound."""
    _case(f"head mix unsupported ({why}) {shape} heads={heads}")
    B, C, H, W = shape
    sh = _table("half6")
    x, hw, mix = _inputs(torch.float32, shape, sh.size(0), heads, 9)
    assert _C.normalized_accumulate_uz_forward_mixed(x.to(DEV), hw.to(DEV), mix,
                                                     sh.to(DEV)) is None
    assert "heads" in _C._lib.nsh_last_error().decode() or why == "shape"
    with torch.no_grad():
        D, L = normalized_accumulate_uz_mixed(x.to(DEV), hw.to(DEV), mix.to(DEV), sh.to(DEV),
                                              return_log_degree=True)
    wo = _oracle_weights(hw, mix, C, torch.float32)
    Do, Lo = oracle.normalized(x, wo, sh, log_weights=False, policy="gpu")
    Ds, _ = oracle.normalized(x.abs(), wo, sh, log_weights=False, policy="gpu")
    assert_bound(D, Do, Ds, rtol_for(torch.float32), "D")
    assert_bound(L, Lo, Lo.abs().nan_to_num(posinf=0, neginf=0) + 1.0, rtol_for(torch.float32),
                 "log_C")


def test_mixed_forward_rejects_bad_arguments():
    _case("head mix argument checks")
    sh = _table("half6").to(DEV)
    x, hw, mix = _inputs(torch.float32, (1, 3, 72, 200), sh.size(0), 2, 3)
    with pytest.raises(RuntimeError, match="head_mix must be"):
        _C.normalized_accumulate_uz_forward_mixed(x.to(DEV), hw.to(DEV), mix[:2], sh)
    with pytest.raises(RuntimeError, match="head_weights must be"):
        _C.normalized_accumulate_uz_forward_mixed(x.to(DEV), hw[:-1].to(DEV), mix, sh)
    with pytest.raises(ValueError, match="head_mix must be"):
        normalized_accumulate_uz_mixed(x.to(DEV), hw.to(DEV), mix[:, :1].to(DEV), sh)


def test_mixed_forward_autograd_route():
    """With a gradient wanted the op mixes first: the same values as the
    plain op on the matmul-mixed weights, and gradients reach the heads and
    the matrix."""
    _case("head mix autograd route")
    sh = _table("half6").to(DEV)
    S = sh.size(0)
    x, hw, mix = _inputs(torch.float32, (1, 3, 72, 200), S, 2, 13)
    hwd = hw.to(DEV).requires_grad_(True)
    mixd = mix.float().to(DEV).requires_grad_(True)
    D = normalized_accumulate_uz_mixed(x.to(DEV), hwd, mixd, sh)
    # the op's mixing product, as the op forms it (ops.mix_head_planes: the HIP kernels)
    from neural_shift_cuda_amd.ops import mix_head_planes
    with torch.no_grad():
        mixed = mix_head_planes(hwd.detach().reshape(S, 2, -1), mixd.detach())
    mixed = mixed.view(S, 3, 72, 200)
    Dr = normalized_accumulate_uz(x.to(DEV), mixed, sh, validate=False)
    assert torch.equal(D.detach(), Dr)
    D.sum().backward()
    assert hwd.grad is not None and torch.isfinite(hwd.grad).all()
    assert mixd.grad is not None and torch.isfinite(mixd.grad).all()
    with torch.no_grad():
        Df = normalized_accumulate_uz_mixed(x.to(DEV), hwd, mixd, sh)
    assert_bound(Df, Dr.double().cpu(), Dr.abs().double().cpu() + x.abs().amax().item(),
                 2 * rtol_for(torch.float32), "no-grad fused vs autograd route")


@pytest.mark.parametrize("kind,comp_box", [("nekde", True), ("nekde", False), ("gasd", True)])
def test_installers_fused_forward(kind, comp_box, monkeypatch):
    """The installed forward of two-head stand-in models on an image the
    scatter path serves (two 128-pixel fp32 tiles across): without autograd
    (the fused op, which must have served the call) against the same
    forward with autograd (mixing first)."""
    from installer_models import FakeGASD, FakeNeKDe, _fresh, _inputs as model_inputs
    from neural_shift_cuda.integration import install_cuda_shift_attn, install_cuda_shift_gasd
    _case(f"installed {kind} fused head mix comp_box={comp_box}")
    cls, install = ((FakeNeKDe, install_cuda_shift_attn) if kind == "nekde"
                    else (FakeGASD, install_cuda_shift_gasd))
    sub, m = _fresh(cls, comp_box=comp_box, heads=2)
    x, guide = model_inputs(H=72, W=200)
    install(sub)
    m = m.to(device="cuda", dtype=torch.float32)
    xc, gc = x.float().cuda(), guide.float().cuda()
    served = []
    fused = _C.normalized_accumulate_uz_forward_mixed
    monkeypatch.setattr(_C, "normalized_accumulate_uz_forward_mixed",
                        lambda *a, **k: served.append(fused(*a, **k)) or served[-1])
    D, Z = m.forward(xc, guide=gc)           # parameters require grad: mixing first
    assert not served
    with torch.no_grad():
        Df, Zf = m.forward(xc, guide=gc)     # the fused op
    assert len(served) == 1 and served[0] is not None
    scale = D.detach().abs() + xc.abs().amax()
    assert_bound(Df, D.detach().double().cpu(), scale.double().cpu(),
                 2 * rtol_for(torch.float32), "D fused vs mixed first")
    assert_bound(Zf, Z.detach().double().cpu(), Z.detach().abs().double().cpu(),
                 2 * rtol_for(torch.float32), "Z fused vs mixed first")


# ---------------------------------------------------------------------------
# The mixing product itself on the GPU (training path): nsh_head_mix_forward
# and nsh_head_mix_backward through ops.mix_head_planes, against fp64.
# Bounds: the rule of tests/helpers.py with the term scale of each sum (the
# same sum over absolute values) and the output rounding of 16-bit outputs;
# the matrix gradient sums N*P terms through a two-level reduction whose
# longest sequential chain is below 100 additions (well inside 1e-5 / u).
# ---------------------------------------------------------------------------

MIX_CASES = [
    (torch.float32, 2, 3, 40, 65536),   # 16-byte vectors
    (torch.float32, 4, 8, 300, 65536),  # planes looped (300 > 16384 / 64 workgroups)
    (torch.float32, 3, 1, 17, 4097),    # P not a vector multiple: 1-element lanes
    (torch.float16, 3, 3, 24, 32768),
    (torch.bfloat16, 2, 5, 24, 8192),
    (torch.float64, 4, 3, 12, 16384),
    (torch.float64, 2, 2, 7, 1001),
]


@pytest.mark.parametrize("dtype,heads,C,N,P", MIX_CASES)
def test_head_mix_kernels_vs_fp64(dtype, heads, C, N, P):
    from helpers import out_ulp_for
    from neural_shift_cuda_amd.ops import mix_head_planes
    _case(f"head mix kernels {dtype} heads={heads} C={C} N={N} P={P}")
    g = torch.Generator().manual_seed(heads * 100 + C)
    acc = torch.float64 if dtype == torch.float64 else torch.float32
    w = torch.randn(N, heads, P, generator=g).to(dtype)
    mix = torch.randn(C, heads, generator=g, dtype=torch.float64).to(acc)
    go = torch.randn(N, C, P, generator=g).to(dtype)
    wd = w.to(DEV).requires_grad_(True)
    md = mix.to(DEV).requires_grad_(True)
    out = mix_head_planes(wd, md)
    out.backward(go.to(DEV))
    torch.cuda.synchronize()
    rt, ou = rtol_for(dtype), out_ulp_for(dtype)
    w64, m64, g64 = w.double(), mix.double(), go.double()
    ref = torch.einsum("ch,nhp->ncp", m64, w64)
    sc = torch.einsum("ch,nhp->ncp", m64.abs(), w64.abs())
    assert_bound(out.detach(), ref, sc, rt, "out", ou)
    gw_ref = torch.einsum("ch,ncp->nhp", m64, g64)
    gw_sc = torch.einsum("ch,ncp->nhp", m64.abs(), g64.abs())
    assert_bound(wd.grad, gw_ref, gw_sc, rt, "grad_w", ou)
    gm_ref = torch.einsum("ncp,nhp->ch", g64, w64)
    gm_sc = torch.einsum("ncp,nhp->ch", g64.abs(), w64.abs())
    assert_bound(md.grad, gm_ref, gm_sc, rt, "grad_mix")


def test_head_mix_kernels_deterministic_and_unsupported():
    from neural_shift_cuda_amd.ops import mix_head_planes
    _case("head mix kernels determinism, unsupported counts")
    g = torch.Generator().manual_seed(3)
    w = torch.randn(50, 3, 20000, generator=g).to(DEV)
    mix = torch.randn(3, 3, generator=g).to(DEV)
    go = torch.randn(50, 3, 20000, generator=g).to(DEV)
    runs = [_C.head_mix_backward(w, mix, go) for _ in range(2)]
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    assert _C.head_mix_forward(torch.randn(4, 5, 64, device=DEV), torch.randn(3, 5)) is None
    assert _C.head_mix_forward(torch.randn(4, 2, 64, device=DEV), torch.randn(9, 2)) is None
    # the op takes the broadcast form for those counts
    w5 = torch.randn(4, 5, 64, generator=g).to(DEV)
    m5 = torch.randn(3, 5, generator=g).to(DEV)
    ref = torch.einsum("ch,nhp->ncp", m5.double(), w5.double())
    assert_bound(mix_head_planes(w5, m5), ref.cpu(),
                 torch.einsum("ch,nhp->ncp", m5.double().abs(), w5.double().abs()).cpu(),
                 rtol_for(torch.float32), "broadcast form")
