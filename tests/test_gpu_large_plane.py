"""accumulate_uz on a plane just under the 2^31-byte in-plane limit.

The kernels address the weight and weight-gradient planes as a uniform base
plus the lane's 32-bit byte offset (buffer accesses) and the other planes with
32-bit in-plane offsets; the host rejects a (b, c) plane of 2^31 bytes or more
(tests/test_abi.py checks the rejection).
Here one fp32 plane is 23168 x 23168 = 2,147,024,896 bytes, 458,752 bytes
short of the limit, so the last pixels' byte offsets lie just under 2^31:
forward and backward run through the scatter path (workspace from the
package), and crops, among them the bottom-right corner where the offsets are
largest and crops across the wrap, are compared with the window oracle (the
global wrap and box rules of the whole image) at the accumulation bound
(rtol 1e-5 of the per-element absolute-value sum).  About 36 GB of device
memory.
"""
from __future__ import annotations

import sys

import pytest
import torch

import oracle
from helpers import assert_bound
from neural_shift_cuda import accumulate_uz
from neural_shift_cuda_amd.workloads import box_stack, halfplane_shifts

HAS_GPU = torch.cuda.is_available()
DEV = torch.device("cuda:0")


def _case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _setup():
    oracle.build()


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
def test_gpu_accumulate_plane_near_2gib():
    B, C, H, W, R = 1, 1, 23168, 23168, 1
    assert (2 ** 31) - 2 ** 20 < H * W * 4 < 2 ** 31
    sh = halfplane_shifts(R)
    S = sh.size(0)
    _case(f"accumulate_uz fwd+bwd fp32 {B}x{C}x{H}x{W} S={S} (plane {H * W * 4} bytes)")
    g = torch.Generator(device=DEV).manual_seed(611)
    x = torch.rand(B, C, H, W, generator=g, device=DEV)
    w = torch.empty(S * B, C, H, W, device=DEV)
    for s in range(S):
        blk = torch.nn.functional.softplus(torch.randn(B, C, H, W, generator=g, device=DEV))
        w[s * B:(s + 1) * B] = blk * box_stack(sh[s:s + 1], 1, H, W, device=DEV)
    gU = torch.randn(B, C, H, W, generator=g, device=DEV)
    gZ = torch.randn(B, C, H, W, generator=g, device=DEV)
    x.requires_grad_(True)
    w.requires_grad_(True)
    U, Z = accumulate_uz(x, w, sh.to(DEV))
    torch.autograd.backward([U, Z], [gU, gZ])
    torch.cuda.synchronize()
    ch = cw = 64
    crops = [(H - ch, W - cw),            # last rows and columns: the largest offsets
             (H - ch - 8, W - cw - 8),    # interior, next to them
             (H - ch // 2, W - cw // 2),  # across the wrap at the far corner
             (0, 0), (H // 2, W // 3), (17, W - 40)]
    xs, ws = x.detach(), w.detach()
    for k, (gh0, gw0) in enumerate(crops):
        _case(f"crop {k} at {(gh0, gw0)}")
        win = lambda t: oracle.take_window(t, gh0, gw0, ch, cw, R)
        crop = lambda t: oracle.take_window(t, gh0, gw0, ch, cw, 0)
        xw, ww, gUw, gZw = win(xs), win(ws), win(gU), win(gZ)
        Uo, Zo = oracle.accumulate_uz_window(xw, ww, sh, R, H, W, gh0, gw0, ch, cw)
        Us, Zs = oracle.accumulate_uz_window(xw.abs(), ww.abs(), sh, R, H, W, gh0, gw0, ch, cw)
        assert_bound(crop(U.detach()), Uo, Us, 1e-5, f"U crop {k}")
        assert_bound(crop(Z.detach()), Zo, Zs, 1e-5, f"Z crop {k}")
        gxo, gwo = oracle.accumulate_uz_window_bwd(xw, ww, gUw, gZw, sh, R, H, W, gh0, gw0, ch, cw)
        gxs, gws = oracle.accumulate_uz_window_bwd(xw.abs(), ww.abs(), gUw.abs(), gZw.abs(), sh,
                                                   R, H, W, gh0, gw0, ch, cw)
        assert_bound(crop(x.grad), gxo, gxs, 1e-5, f"grad_x crop {k}")
        assert_bound(crop(w.grad), gwo, gws, 1e-5, f"grad_w crop {k}")
    del x, w, U, Z, gU, gZ, xs, ws
    torch.cuda.empty_cache()
