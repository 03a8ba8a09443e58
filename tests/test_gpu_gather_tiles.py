"""shift_gather / pair_gather on shapes that take the tiled kernels (16-byte
vectors: W a multiple of 8 / 4 / 2 elements for 16-bit / fp32 / fp64,
aligned tensors), against the CPU oracle: the forward bit-exact (values and
mask), the backward to the accumulation tolerance and bitwise deterministic.

Tiles are 8 rows x min(W, 256) columns with an 8-pixel LDS halo; the shapes
cover partial tiles in both directions, images narrower than a tile and
shorter than the halo (multiple wraps), several column tiles, and tables
with shifts beyond the halo in either direction (element-wise path) and
larger than the image (modular reduction).
"""
from __future__ import annotations

import sys

import pytest
import torch

import oracle
from helpers import assert_bound, out_ulp_for, rtol_for
from neural_shift_cuda import pair_gather, shift_gather
from neural_shift_cuda_amd.workloads import halfplane_shifts, window_shifts

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
        "half5": halfplane_shifts(5),
        "win8": window_shifts(8),
        "far": torch.tensor([[0, 0, 0], [9, 3, 1], [-2, 11, 1], [1, -10, 1], [3, 2, 0],
                             [-20, -9, 0], [40, 70, 1]]),
    }[name]


SHAPES = [(2, 3, 37, 264), (1, 2, 5, 8), (1, 1, 19, 520), (3, 1, 64, 64)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32, torch.float64])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("table", ["half5", "win8", "far"])
def test_gather_tiles_forward_bit_exact(dtype, shape, table):
    _case(f"gather tiles fwd {dtype} {shape} {table}")
    B, C, H, W = shape
    g = torch.Generator().manual_seed(11)
    guide = torch.randn(B, C, H, W, generator=g).to(dtype)
    sh = _table(table)
    gs, m = shift_gather(guide.to(DEV), sh.to(DEV))
    go, mo = oracle.shift_gather(guide, sh)
    assert torch.equal(gs.cpu(), go) and torch.equal(m.cpu(), mo)
    p, pm = pair_gather(guide.to(DEV), sh.to(DEV))
    po, pmo = oracle.pair_gather(guide, sh)
    assert torch.equal(p.cpu(), po) and torch.equal(pm.cpu(), pmo)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float64])
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("table", ["half5", "far"])
@pytest.mark.parametrize("pair", [False, True])
def test_gather_tiles_backward(dtype, shape, table, pair):
    _case(f"gather tiles bwd {dtype} {shape} {table} pair={pair}")
    B, C, H, W = shape
    g = torch.Generator().manual_seed(12)
    sh = _table(table)[:, :2].contiguous()
    guide = torch.randn(B, C, H, W, generator=g).to(dtype).to(DEV).requires_grad_(True)
    fn = pair_gather if pair else shift_gather
    out, _ = fn(guide, sh.to(DEV))
    gout = torch.randn(out.shape, generator=g).to(dtype)
    out.backward(gout.to(DEV))
    bwd = oracle.pair_gather_bwd if pair else oracle.shift_gather_bwd
    ref = bwd(gout, sh, B, C, H, W)
    scale = bwd(gout.abs(), sh, B, C, H, W)
    assert_bound(guide.grad, ref, scale, rtol_for(dtype), "grad_guide", out_ulp_for(dtype))
    g1 = guide.grad.clone()
    guide.grad = None
    out, _ = fn(guide, sh.to(DEV))
    out.backward(gout.to(DEV))
    assert torch.equal(g1, guide.grad)  # deterministic, atomic-free
