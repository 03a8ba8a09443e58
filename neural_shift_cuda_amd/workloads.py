"""Shift tables and seeded synthetic inputs for the shift-window ops.

Shift tables follow the reference's conventions:
  * ``halfplane_shifts(R)``: the canonical half-plane with mirror flags,
    (dx in [-R, R], dy in [1, R], inv 1) then (dx in [0, R], 0, inv dx != 0)
    (nectr_patch.py:55-69, tests/test_accumulate_uz.py:12-19); S = 2R^2+2R+1.
  * ``window_shifts(R)``: the full (2R+1)^2 window with has_inverse = 0
    (gasd_drunet_attn_patch.py:88-103).
  * ``explicit_mirror_shifts(table)``: a half-plane table in "periodic" form,
    every mirror written out as its own has_inverse = 0 row
    (nekde_drunet_attn_patch.py:350-366).

``synthetic_image`` draws the piecewise-smooth test image of the benchmark
configurations: 8 axis-aligned rectangles with U[0, 1] intensities painted in
order, plus 0.1 sin(2 pi (f_h h / H + f_w w / W) + phi) with f ~ U[1, 8],
phi ~ U[0, 2 pi), plus iid N(0, (25/255)^2) noise; channels independent.
All randomness comes from a CPU ``torch.Generator``.
"""
from __future__ import annotations

import math
from typing import List, Sequence, Tuple

import torch


def halfplane_rows(R: int) -> List[Tuple[int, int, int]]:
    rows = [(dx, dy, 1) for dx in range(-R, R + 1) for dy in range(1, R + 1)]
    rows += [(dx, 0, 0 if dx == 0 else 1) for dx in range(0, R + 1)]
    return rows


def halfplane_shifts(R: int, dtype=torch.int64) -> torch.Tensor:
    return torch.tensor(halfplane_rows(R), dtype=dtype)


def window_shifts(R: int, with_flag: bool = True, dtype=torch.int64) -> torch.Tensor:
    rows = [(dx, dy, 0) if with_flag else (dx, dy)
            for dx in range(-R, R + 1) for dy in range(-R, R + 1)]
    return torch.tensor(rows, dtype=dtype)


def explicit_mirror_shifts(table: torch.Tensor) -> torch.Tensor:
    rows = []
    for dx, dy, inv in table.tolist():
        rows.append((dx, dy, 0))
        if inv:
            rows.append((-dx, -dy, 0))
    return torch.tensor(rows, dtype=table.dtype)


def box_stack(shifts: torch.Tensor, B: int, H: int, W: int, dtype=torch.float32,
              device="cpu") -> torch.Tensor:
    """(S*B, 1, H, W) forward box of every shift row, shift-major."""
    out = []
    hs = torch.arange(H, device=device)
    ws = torch.arange(W, device=device)
    for dx, dy in shifts[:, :2].tolist():
        r = ((hs + dx) >= 0) & ((hs + dx) < H)
        c = ((ws + dy) >= 0) & ((ws + dy) < W)
        out.append((r[:, None] & c[None, :]).to(dtype).expand(B, 1, H, W))
    return torch.cat(out, 0)


def synthetic_image(B: int, C: int, H: int, W: int, seed: int,
                    dtype=torch.float32) -> torch.Tensor:
    """Piecewise-smooth seeded image (see module docstring), on the CPU."""
    g = torch.Generator().manual_seed(seed)
    img = torch.zeros(B, C, H, W, dtype=torch.float32)
    hh = torch.arange(H, dtype=torch.float32)[:, None] / H
    ww = torch.arange(W, dtype=torch.float32)[None, :] / W
    for b in range(B):
        for c in range(C):
            plane = img[b, c]
            for _ in range(8):
                h0, h1 = sorted(torch.randint(0, H + 1, (2,), generator=g).tolist())
                w0, w1 = sorted(torch.randint(0, W + 1, (2,), generator=g).tolist())
                plane[h0:h1, w0:w1] = torch.rand((), generator=g).item()
            fh, fw = (1.0 + 7.0 * torch.rand(2, generator=g)).tolist()
            phi = 2.0 * math.pi * torch.rand((), generator=g).item()
            plane += 0.1 * torch.sin(2.0 * math.pi * (fh * hh + fw * ww) + phi)
    img += (25.0 / 255.0) * torch.randn(B, C, H, W, generator=g)
    return img.to(dtype)


def softplus_weights(shape: Sequence[int], seed: int, dtype=torch.float32,
                     device="cpu") -> torch.Tensor:
    """softplus(N(0, 1)) weights, drawn on `device` from a seeded generator."""
    g = torch.Generator(device=device).manual_seed(seed)
    w = torch.randn(*shape, generator=g, device=device, dtype=torch.float32)
    return torch.nn.functional.softplus(w).to(dtype)


def logit_weights(shape: Sequence[int], seed: int, dtype=torch.float32,
                  device="cpu", outlier_frac: float = 0.01, outlier: float = 80.0
                  ) -> torch.Tensor:
    """Logits N(0, variance 4) with a seeded fraction set to +-outlier."""
    g = torch.Generator(device=device).manual_seed(seed)
    z = 2.0 * torch.randn(*shape, generator=g, device=device, dtype=torch.float32)
    pick = torch.rand(*shape, generator=g, device=device) < outlier_frac
    sign = torch.where(torch.rand(*shape, generator=g, device=device) < 0.5, -1.0, 1.0)
    z = torch.where(pick, sign * outlier, z)
    return z.to(dtype)


# fp32, B=1, C=1, H=W=256, R=3 half-plane (S=25),
# comp_box=True, the piecewise-smooth image, softplus(N(0,1)) weights
# multiplied by the forward box (reference ops.py:619-620).
C0_SHAPE = (1, 1, 256, 256)
C0_RADIUS = 3
C0_SEEDS = (1, 2)


def config0_inputs():
    """(x, w, shifts) of configuration c0 on the CPU, fp32."""
    B, C, H, W = C0_SHAPE
    sh = halfplane_shifts(C0_RADIUS)
    x = synthetic_image(B, C, H, W, seed=C0_SEEDS[0])
    w = softplus_weights((sh.size(0) * B, C, H, W), seed=C0_SEEDS[1])
    w = w * box_stack(sh, B, H, W)
    return x, w, sh


def tensor_digest(*tensors: torch.Tensor) -> str:
    """sha256 of the tensors' bytes (shape and dtype included), to tie
    stored outputs to regenerated inputs."""
    import hashlib
    h = hashlib.sha256()
    for t in tensors:
        t = t.detach().contiguous().cpu()
        h.update(f"{tuple(t.shape)}{t.dtype}".encode())
        h.update(t.view(torch.uint8).numpy().tobytes() if t.dtype != torch.bool
                 else t.numpy().tobytes())
    return h.hexdigest()
