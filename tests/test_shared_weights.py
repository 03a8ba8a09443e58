"""Channel-shared weights (``shared_weights=True``: weights (S*B, 1, H, W)
used for every channel, the single-head weights the reference installers
broadcast before the ops, nekde_drunet_attn_patch.py:117-140).

The pin is the same op on the broadcast weights materialised per channel:
values and x gradients equal, and the shared weights' gradient equals the
sum over the channels of the per-channel weight gradient.  On the GPU the
HIP kernels read the shared plane (NSH_SHARED_WEIGHTS), on the CPU the
fallbacks run on the expanded view.
"""
from __future__ import annotations

import sys

import pytest
import torch

import oracle
from helpers import assert_bound, normalized_bwd_cond, out_ulp_for, rtol_for
from neural_shift_cuda import accumulate_uz, normalized_accumulate_uz
from neural_shift_cuda_amd import _C
from neural_shift_cuda_amd.workloads import halfplane_shifts, window_shifts

HAS_GPU = torch.cuda.is_available()
DEV = torch.device("cuda:0")


def _case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _inputs(B, C, H, W, S, dtype, seed, positive=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, C, H, W, generator=g).to(dtype)
    w = torch.randn(S * B, 1, H, W, generator=g)
    w = (torch.nn.functional.softplus(w) if positive else 2 * w).to(dtype)
    acc = torch.float64 if dtype == torch.float64 else torch.float32
    gU = torch.randn(B, C, H, W, generator=g).to(acc)
    gZ = torch.randn(B, C, H, W, generator=g).to(acc)
    return x, w, gU, gZ


@pytest.mark.parametrize("normalized", [False, True])
def test_cpu_shared_equals_broadcast(normalized):
    sh = halfplane_shifts(2)
    B, C, H, W = 2, 3, 9, 11
    x, w, gU, gZ = _inputs(B, C, H, W, sh.size(0), torch.float64, 1)
    xs, ws = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    xe, we = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    if normalized:
        a = normalized_accumulate_uz(xs, ws, sh, return_log_degree=True, shared_weights=True)
        b = normalized_accumulate_uz(xe, we.expand(-1, C, -1, -1).contiguous(), sh,
                                     return_log_degree=True)
    else:
        a = accumulate_uz(xs, ws, sh, shared_weights=True)
        b = accumulate_uz(xe, we.expand(-1, C, -1, -1).contiguous(), sh)
    torch.autograd.backward(list(a), [gU, gZ])
    torch.autograd.backward(list(b), [gU, gZ])
    for u, v in zip(a, b):
        torch.testing.assert_close(u, v, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(xs.grad, xe.grad, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(ws.grad, we.grad, rtol=1e-12, atol=1e-12)
    with pytest.raises(ValueError, match="shared weights"):
        accumulate_uz(x, w.expand(-1, C, -1, -1), sh, shared_weights=True)


# (shape, dtype, table): scatter-path shapes (>= 3 tiles per direction) and
# one that takes the gather kernels
GPU_CASES = [
    ((1, 3, 72, 200), torch.float32, "half3"),
    ((2, 3, 104, 136), torch.float16, "half6"),
    ((1, 2, 104, 104), torch.float64, "win2"),
    ((2, 3, 30, 44), torch.float32, "half3"),
]


def _channel_rounding(dtype, C):
    """Absolute error of rounding each of the C per-channel weight gradients
    to the weights' dtype before their sum, where the relative bound does not
    hold: half a subnormal step per channel."""
    fi = torch.finfo(dtype)
    return C * fi.tiny * fi.eps / 2


def _table(name):
    return {"half3": halfplane_shifts(3), "half6": halfplane_shifts(6),
            "win2": window_shifts(2)}[name]


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
@pytest.mark.parametrize("shape,dtype,table", GPU_CASES)
@pytest.mark.parametrize("opts", [{}, {"box_forward": True}, {"periodic_inverse": True}])
def test_gpu_accumulate_shared_weights(shape, dtype, table, opts):
    _case(f"shared accumulate {shape} {dtype} {table} {opts}")
    sh = _table(table)
    B, C, H, W = shape
    x, w, gU, gZ = _inputs(B, C, H, W, sh.size(0), dtype, 2)
    xd, wd = x.to(DEV).requires_grad_(True), w.to(DEV).requires_grad_(True)
    U, Z = accumulate_uz(xd, wd, sh.to(DEV), shared_weights=True, **opts)
    torch.autograd.backward([U, Z], [gU.to(DEV), gZ.to(DEV)])
    # the same op on the materialised broadcast, on the GPU
    xe = x.to(DEV).requires_grad_(True)
    we = w.to(DEV).expand(-1, C, -1, -1).contiguous().requires_grad_(True)
    Ue, Ze = accumulate_uz(xe, we, sh.to(DEV), **opts)
    torch.autograd.backward([Ue, Ze], [gU.to(DEV), gZ.to(DEV)])
    torch.cuda.synchronize()
    assert torch.equal(U, Ue) and torch.equal(Z, Ze)
    assert torch.equal(xd.grad, xe.grad)
    assert wd.grad.shape == w.shape
    rt = rtol_for(dtype)
    ou = out_ulp_for(dtype)
    ge = we.grad.double().cpu()
    assert_bound(wd.grad, ge.sum(1, keepdim=True), ge.abs().sum(1, keepdim=True), rt,
                 "grad_w vs the channel sum", 2 * ou)
    # the oracle's per-channel gradient, summed over the channels
    wx = w.expand(-1, C, -1, -1).contiguous()
    if not opts:
        Uo, Zo = oracle.accumulate_uz(x, wx, sh)
        Us, Zs = oracle.accumulate_uz(x.abs(), wx.abs(), sh)
        assert_bound(U, Uo, Us, rt, "U")
        assert_bound(Z, Zo, Zs, rt, "Z")
        gxo, gwo = oracle.accumulate_uz_bwd(x, wx, gU, gZ, sh)
        gxs, gws = oracle.accumulate_uz_bwd(x.abs(), wx.abs(), gU.abs(), gZ.abs(), sh)
        assert_bound(xd.grad, gxo, gxs, rt, "grad_x", ou)
        # each channel's gradient is rounded to the weights' dtype before the
        # sum: up to out_ulp of each channel's magnitude (<= the scale)
        gsc = gws.sum(1, keepdim=True)
        assert_bound(wd.grad, gwo.sum(1, keepdim=True), gsc, rt, "grad_w (sum over channels)",
                     2 * ou, extra=ou * gsc + _channel_rounding(dtype, C))


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
@pytest.mark.parametrize("shape,dtype,table", GPU_CASES)
@pytest.mark.parametrize("log_weights", [False, True])
def test_gpu_normalized_shared_weights(shape, dtype, table, log_weights):
    _case(f"shared normalized {shape} {dtype} {table} log={log_weights}")
    sh = _table(table)
    B, C, H, W = shape
    x, w, gD, gL = _inputs(B, C, H, W, sh.size(0), dtype, 3, positive=not log_weights)
    xd, wd = x.to(DEV).requires_grad_(True), w.to(DEV).requires_grad_(True)
    D, L = normalized_accumulate_uz(xd, wd, sh.to(DEV), log_weights=log_weights,
                                    return_log_degree=True, shared_weights=True)
    torch.autograd.backward([D, L], [gD.to(DEV), gL.to(DEV)])
    xe = x.to(DEV).requires_grad_(True)
    we = w.to(DEV).expand(-1, C, -1, -1).contiguous().requires_grad_(True)
    De, Le = normalized_accumulate_uz(xe, we, sh.to(DEV), log_weights=log_weights,
                                      return_log_degree=True)
    torch.autograd.backward([De, Le], [gD.to(DEV), gL.to(DEV)])
    torch.cuda.synchronize()
    assert torch.equal(D, De) and torch.equal(L, Le)
    assert torch.equal(xd.grad, xe.grad)
    # oracle: values and the channel sum of the weight gradient
    rt = rtol_for(dtype)
    wx = w.expand(-1, C, -1, -1).contiguous()
    Do, Lo = oracle.normalized(x, wx, sh, log_weights=log_weights, policy="gpu")
    Ds, _ = oracle.normalized(x.abs(), wx, sh, log_weights=log_weights, policy="gpu")
    assert_bound(D, Do, Ds, rt, "D")
    gxo, gwo = oracle.normalized_bwd(x, wx, Do, Lo, gD, gL, sh, log_weights=log_weights)
    gxs, gws = oracle.normalized_bwd(x.abs(), wx, -Ds, Lo, gD.abs(), gL.abs(), sh,
                                     log_weights=log_weights)
    gxc, gwc = normalized_bwd_cond(x, wx, Lo, gD, gL, Ds, sh, log_weights=log_weights,
                                   acc_dtype=dtype)
    ou = out_ulp_for(dtype)
    assert_bound(xd.grad, gxo, gxs, rt, "grad_x", ou, extra=gxc)
    gsc = gws.sum(1, keepdim=True)
    assert_bound(wd.grad, gwo.sum(1, keepdim=True), gsc, rt, "grad_w (sum over channels)",
                 2 * ou, extra=gwc.sum(1, keepdim=True) + ou * gsc + _channel_rounding(dtype, C))
    ge = we.grad.double().cpu()
    assert_bound(wd.grad, ge.sum(1, keepdim=True), ge.abs().sum(1, keepdim=True), rt,
                 "grad_w vs the channel sum", 2 * ou)


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
def test_gpu_shared_weights_c_abi_flag():
    """The C ABI reads a (S*B, 1, H, W) tensor under NSH_SHARED_WEIGHTS."""
    _case("shared weights C ABI")
    sh = halfplane_shifts(3).to(DEV)
    B, C, H, W = 1, 3, 72, 200
    x, w, _, _ = _inputs(B, C, H, W, sh.size(0), torch.float32, 4)
    U, Z = _C.accumulate_uz_forward(x.to(DEV), w.to(DEV), sh, shared_weights=True)
    Ue, Ze = _C.accumulate_uz_forward(x.to(DEV), w.expand(-1, C, -1, -1).contiguous().to(DEV), sh)
    assert torch.equal(U, Ue) and torch.equal(Z, Ze)
    with pytest.raises(RuntimeError, match="weights shape must be"):
        _C.accumulate_uz_forward(x.to(DEV), w.to(DEV), sh)
    with pytest.raises(RuntimeError, match="shared weights must be"):
        _C.accumulate_uz_forward(x.to(DEV), w.expand(-1, C, -1, -1).contiguous().to(DEV), sh,
                                 shared_weights=True)
