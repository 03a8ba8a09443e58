"""normalized_accumulate_uz_mixed on the CPU: the heads are mixed first
(the installers' product, reference nekde_drunet_attn_patch.py:117-140) and
the normalized accumulation's CPU fallback runs on the result, so the op is
that composition (the mixing summed as a broadcast product: to the last
bits of an fp64 matmul); argument checks.  The in-kernel mixing is tested
on the GPU (tests/test_gpu_head_mix.py)."""
from __future__ import annotations

import pytest
import torch

from neural_shift_cuda_amd.ops import normalized_accumulate_uz, normalized_accumulate_uz_mixed
from neural_shift_cuda_amd.workloads import halfplane_shifts


@pytest.mark.parametrize("heads,box,periodic", [(2, False, False), (3, True, False),
                                                (4, False, True)])
def test_mixed_cpu_is_mix_then_normalized(heads, box, periodic):
    g = torch.Generator().manual_seed(heads)
    sh = halfplane_shifts(2)
    S, B, C, H, W = sh.size(0), 2, 3, 9, 11
    x = torch.randn(B, C, H, W, generator=g, dtype=torch.float64)
    hw = torch.rand(S * B, heads, H, W, generator=g, dtype=torch.float64)
    mix = torch.softmax(torch.randn(C, heads, generator=g, dtype=torch.float64), dim=1)
    D, L = normalized_accumulate_uz_mixed(x, hw, mix, sh, return_log_degree=True,
                                          box_forward=box, periodic_inverse=periodic)
    mixed = torch.matmul(mix, hw.reshape(S * B, heads, H * W)).view(S * B, C, H, W)
    Dr, Lr = normalized_accumulate_uz(x, mixed, sh, return_log_degree=True, validate=False,
                                      box_forward=box, periodic_inverse=periodic)
    torch.testing.assert_close(D, Dr, rtol=1e-13, atol=1e-15)
    torch.testing.assert_close(L, Lr, rtol=1e-13, atol=1e-15)
    assert torch.equal(normalized_accumulate_uz_mixed(x, hw, mix, sh, box_forward=box,
                                                      periodic_inverse=periodic), D)


def test_mixed_argument_checks():
    sh = halfplane_shifts(1)
    x = torch.rand(1, 3, 5, 6, dtype=torch.float64)
    hw = torch.rand(sh.size(0), 2, 5, 6, dtype=torch.float64)
    with pytest.raises(ValueError, match="head_mix must be"):
        normalized_accumulate_uz_mixed(x, hw, torch.rand(2, 2, dtype=torch.float64), sh)
    with pytest.raises(ValueError, match="head_weights must be"):
        normalized_accumulate_uz_mixed(x, hw[0], torch.rand(3, 2, dtype=torch.float64), sh)
