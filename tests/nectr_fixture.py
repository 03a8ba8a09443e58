"""A stand-in for the official NECTR denoiser (reference
models/NECTR_models1.py:12-244), built from the golden case's
configuration with the same parameter names, so that the parameters the
golden generator stored load into it.  Its unpatched forward restates the
model's serial half-plane loop with torch.roll; the golden vectors pin it to
the model's own output.

Architecture (model_type 'concat'):
  guide = pre_activation(x):  [x, sigma map if not blind] -> in_layer
          (patch conv) -> residual_depth x (x + in_residual[i](x), then a
          LayerNorm over channels); in_proj exists but is unused
  N_theta(g, g_s) = activation(out(proj(cat(g, g_s)))), proj = blocks of
          (1x1 conv halving the channels, channels-last LayerNorm, LeakyReLU);
          activation 'exp': exp(v / sigma^2); 'control_sigmoid':
          softplus(a) / (1 + exp(-sigmoid(b) k)) + 1e-8 over three chunks.
  forward: U, Z over the half-plane with box-masked forward weights and the
          circularly rolled, box-masked mirror weights; returns (U / Z, Z).
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F


def _gather(t, dx, dy):
    return torch.roll(t, shifts=(-dx, -dy), dims=(-2, -1))


def _box(H, W, dx, dy, like):
    hs = torch.arange(H, device=like.device) + dx
    ws = torch.arange(W, device=like.device) + dy
    m = ((hs >= 0) & (hs < H))[:, None] & ((ws >= 0) & (ws < W))[None, :]
    return m.to(like.dtype)


def halfplane(R):
    rows = [(dx, dy, True) for dx in range(-R, R + 1) for dy in range(1, R + 1)]
    return rows + [(dx, 0, dx != 0) for dx in range(R + 1)]


class NECTRGoldenModel(nn.Module):
    def __init__(self, cfg):
        super().__init__()
        self.model_type = "concat"
        self.sigma = 1
        self.blind = bool(cfg["blind"])
        self.window_rad = int(cfg["window_rad"])
        self.output_activation = cfg["output_activation"]
        cin, lat, depth = int(cfg["in_channel"]), int(cfg["latent_dim"]), int(cfg["residual_depth"])
        k = 2 * int(cfg["patch_rad"]) + 1
        self.in_layer = nn.Conv2d(cin if self.blind else cin + 1, lat, k, padding=k // 2)
        self.in_proj = nn.ModuleList(
            [nn.Sequential(nn.Conv2d(lat, lat, 3, padding=1), nn.LeakyReLU())
             for _ in range(depth - 1)] + [nn.Conv2d(lat, lat, 3, padding=1)])
        self.in_residual = nn.ModuleList(
            [nn.Sequential(nn.Conv2d(lat, 4 * lat, 1), nn.LeakyReLU(), nn.Conv2d(4 * lat, lat, 1))
             for _ in range(depth)])
        self.in_norm = nn.ModuleList([nn.LayerNorm(lat) for _ in range(depth)])
        width = 2 * lat
        blocks = []
        for _ in range(int(cfg["proj_depth"])):
            blocks.append(nn.ModuleList([nn.Conv2d(width, width // 2, 1),
                                         nn.LayerNorm(width // 2), nn.LeakyReLU()]))
            width //= 2
        self.proj = nn.ModuleList(blocks)
        out = 3 * cin if self.output_activation == "control_sigmoid" else cin
        self.out = nn.Conv2d(width, out, 1, bias=False)

    def pre_activation(self, x, sigma=None):
        if not self.blind:
            if sigma is None:
                raise ValueError("sigma is None, but blind is False")
            s = torch.as_tensor(sigma, dtype=x.dtype, device=x.device).reshape(-1, 1, 1, 1)
            x = torch.cat((x, s.expand(x.shape[0], 1, x.shape[2], x.shape[3])), dim=1)
        g = self.in_layer(x)
        for res, norm in zip(self.in_residual, self.in_norm):
            g = g + res(g)
            g = norm(g.permute(0, 2, 3, 1)).permute(0, 3, 1, 2)
        return g

    def controlled_sigmoid(self, k, a, b):
        return F.softplus(a) / (1 + torch.exp(-torch.sigmoid(b) * k))

    def N_theta(self, g, g_s):
        v = torch.cat((g, g_s), dim=1)
        for conv, norm, act in self.proj:
            v = act(norm(conv(v).permute(0, 2, 3, 1)).permute(0, 3, 1, 2))
        v = self.out(v)
        if self.output_activation == "exp":
            return torch.exp(v / self.sigma ** 2)
        if self.output_activation == "control_sigmoid":
            k, a, b = torch.chunk(v, 3, dim=1)
            return self.controlled_sigmoid(k, a, b) + 1e-8
        return v

    def forward(self, x, reference=None, sig=None, cache=None, store_cache=False):
        g = self.pre_activation(x if reference is None else reference, sigma=sig)
        H, W = x.shape[-2:]
        U = torch.zeros_like(x)
        Z = torch.zeros_like(x)
        held = {}
        for dx, dy, inv in halfplane(self.window_rad):
            if cache is None:
                w = self.N_theta(g, _gather(g, dx, dy)) * _box(H, W, dx, dy, x)
                held[(dx, dy)] = w
            else:
                w = cache[(dx, dy)]
            U = U + w * _gather(x, dx, dy)
            Z = Z + w
            if inv:
                wi = torch.roll(w, shifts=(dx, dy), dims=(-2, -1)) * _box(H, W, -dx, -dy, x)
                U = U + wi * _gather(x, -dx, -dy)
                Z = Z + wi
        return (U / Z, Z, held) if store_cache else (U / Z, Z)


def from_golden(case):
    """(model, x, sig) of a golden 'nectr_installer' case, fp64 on the CPU."""
    m = NECTRGoldenModel(case).double()
    I = case["inputs"]
    state = {k[len("param."):]: v for k, v in I.items() if k.startswith("param.")}
    m.load_state_dict(state, strict=True)
    return m, I["x"], I.get("sig")
