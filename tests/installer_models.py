"""Stand-in model classes for the installer tests and golden vectors.

Each class states its operator directly in its own methods (per-shift loops
over torch.roll), with the method surface the reference installers call
(nekde_drunet_attn_patch.py:576-662, gasd_drunet_attn_patch.py:621-757,
nkd_metropolis_attn_patch.py:193-255, nectr_patch.py:248-299):
pre_activation, _collect_shifts, _halfplane_weights / _all_shift_weights,
_gather_core or attn_head.logit / attn_head.weight, raw_head_mix with
head_mix_pos_act, window_rad, comp_box, max_batch_shifts.

The module depends on torch only, so that tests/golden/make_golden.py can
load it next to the reference package (it imports
``neural_shift_cuda.metropolis`` lazily, from whichever package of that name
is loaded).
"""
from __future__ import annotations

from types import SimpleNamespace

import torch
import torch.nn as nn
import torch.nn.functional as F


def _shift(t, dx, dy):
    """Gather convention: out[h, w] = t[h + dx, w + dy] circularly."""
    return torch.roll(t, shifts=(-dx, -dy), dims=(-2, -1))


def _box(H, W, dx, dy, like):
    hh = torch.arange(H).view(H, 1) + dx
    ww = torch.arange(W).view(1, W) + dy
    ok = (hh >= 0) & (hh < H) & (ww >= 0) & (ww < W)
    return ok.to(like.dtype).to(like.device)


def _halfplane(R):
    rows = [(dx, dy, True) for dx in range(-R, R + 1) for dy in range(1, R + 1)]
    return rows + [(dx, 0, dx != 0) for dx in range(0, R + 1)]


def _symmetric_serial(x, weights, shifts, use_box):
    """U, Z of the symmetric half-plane operator: forward edges as given,
    mirrors rolled by (dx, dy) and (finite window) masked at -s."""
    H, W = x.shape[-2:]
    U = torch.zeros_like(x)
    Z = torch.zeros_like(x)
    for w, (dx, dy, inv) in zip(weights, shifts):
        U = U + w * _shift(x, dx, dy)
        Z = Z + w
        if inv:
            wi = torch.roll(w, shifts=(dx, dy), dims=(-2, -1))
            if use_box:
                wi = wi * _box(H, W, -dx, -dy, x)
            U = U + wi * _shift(x, -dx, -dy)
            Z = Z + wi
    return U, Z


# ---------------------------------------------------------------------------
# Stand-in models
# ---------------------------------------------------------------------------

class _Features(nn.Module):
    """pre_activation: a fixed 1x1 projection to F features plus sigma."""

    def __init__(self, C, Fdim, seed):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        self.proj = nn.Parameter(torch.randn(Fdim, C, generator=g, dtype=torch.float64) * 0.7)

    def forward(self, x, sigma=None):
        phi = torch.einsum("fc,bchw->bfhw", self.proj.to(x.dtype), x)
        return phi if sigma is None else phi + sigma


class _HeadMixMixin:
    def _setup_heads(self, C, heads, seed, pos_act):
        g = torch.Generator().manual_seed(seed + 1)
        self.n_heads = heads
        self.raw_head_mix = (nn.Parameter(torch.randn(C, heads, generator=g, dtype=torch.float64))
                             if heads not in (1, C) or pos_act != "none" else None)
        if pos_act != "none":
            self.head_mix_pos_act = pos_act

    def _mix(self, w, C):
        """(B, h, H, W) -> (B, C, H, W), the models' per-shift head mixing."""
        h = w.shape[1]
        if h == 1:
            return w.expand(-1, C, -1, -1)
        mat = _mix_matrix(self)
        if mat is not None:
            return torch.einsum("ch,bhij->bcij", mat.to(w.dtype), w)
        if h == C:
            return w
        return w.mean(dim=1, keepdim=True).expand(-1, C, -1, -1)


def _mix_matrix(model):
    if model.raw_head_mix is None:
        return None
    act = getattr(model, "head_mix_pos_act", "softmax")
    if act == "softmax":
        return F.softmax(model.raw_head_mix, dim=1)
    if act == "softplus":
        return F.softplus(model.raw_head_mix)
    return F.relu(model.raw_head_mix)


def _head_scores(phi, phi_s, heads, tau=4.0):
    """(B, h, H, W) similarity logits: feature groups per head."""
    B, Fd, H, W = phi.shape
    d = (phi - phi_s).pow(2).view(B, heads, Fd // heads, H, W).sum(dim=2)
    return -d / tau


class FakeNeKDe(nn.Module, _HeadMixMixin):
    """Half-plane symmetric NLM with per-head attention weights."""

    def __init__(self, C=3, R=2, heads=2, comp_box=True, activation="softmax", legacy=False,
                 pos_act="softmax", seed=0):
        super().__init__()
        self.window_rad = R
        self.comp_box = comp_box
        self.output_activation = activation
        self.features = _Features(C, 2 * heads, seed)
        self._setup_heads(C, heads, seed, pos_act)
        self.max_batch_shifts = None
        self.use_grad_checkpoint = False
        self.legacy = legacy
        if not legacy:
            self._gather_core = True
        else:
            self.attn_head = SimpleNamespace(
                logit=lambda pc, ps, s: _head_scores(pc, ps, heads),
                weight=lambda pc, ps, s: torch.sigmoid(_head_scores(pc, ps, heads)) + 1e-3)

    def pre_activation(self, x, sigma=None):
        return self.features(x, sigma)

    def _collect_shifts(self):
        return _halfplane(self.window_rad)

    def _halfplane_weights(self, phi, padded_phi, sig, shift_list):
        R = self.window_rad
        H, W = phi.shape[-2:]
        scores = [_head_scores(phi, padded_phi[:, :, R + dx:R + dx + H, R + dy:R + dy + W],
                               self.n_heads) for dx, dy, _ in shift_list]
        if self.output_activation == "softmax":
            s = torch.stack(scores, dim=1)
            s = F.softmax(s - s.amax(dim=1, keepdim=True), dim=1)
            return list(s.unbind(dim=1))
        return [torch.sigmoid(t) + 1e-3 for t in scores]

    def _weights(self, x, guide, sig):
        phi = self.pre_activation(x if guide is None else guide, sigma=sig)
        R = self.window_rad
        padded = F.pad(phi, (R, R, R, R), mode="circular")
        shifts = self._collect_shifts()
        C = x.shape[1]
        ws = [self._mix(w, C) for w in self._halfplane_weights(phi, padded, sig, shifts)]
        if self.comp_box:
            H, W = x.shape[-2:]
            ws = [w * _box(H, W, dx, dy, x) for w, (dx, dy, _) in zip(ws, shifts)]
        return ws, shifts

    def forward(self, x, guide=None, sig=None, return_D=True):
        ws, shifts = self._weights(x, guide, sig)
        U, Z = _symmetric_serial(x, ws, shifts, self.comp_box)
        return (U / Z, Z) if return_D else (U / Z, None)

    def _KT_action(self, y, guide=None, sig=None, return_D=False, apply_Dinv=False):
        ws, shifts = self._weights(y, guide, sig)
        U, Z = _symmetric_serial(y, ws, shifts, self.comp_box)
        if apply_Dinv:
            U, _ = _symmetric_serial(y / Z.clamp_min(1e-6), ws, shifts, self.comp_box)
        return (U, Z) if return_D else (U, None)


class FakeGASD(FakeNeKDe):
    """Full-window row-stochastic NLM."""

    def _collect_shifts(self):
        R = self.window_rad
        return [(dx, dy) for dx in range(-R, R + 1) for dy in range(-R, R + 1)]

    def _all_shift_weights(self, phi, padded_phi, sig, shift_list):
        return self._halfplane_weights(phi, padded_phi, sig, [(a, b, 0) for a, b in shift_list])

    def _weights(self, x, guide, sig):
        phi = self.pre_activation(x if guide is None else guide, sigma=sig)
        R = self.window_rad
        padded = F.pad(phi, (R, R, R, R), mode="circular")
        shifts = self._collect_shifts()
        C = x.shape[1]
        ws = [self._mix(w, C) for w in self._all_shift_weights(phi, padded, sig, shifts)]
        if self.comp_box:
            H, W = x.shape[-2:]
            ws = [w * _box(H, W, dx, dy, x) for w, (dx, dy) in zip(ws, shifts)]
        return ws, shifts

    def forward(self, x, guide=None, sig=None, return_D=True):
        ws, shifts = self._weights(x, guide, sig)
        U = sum(w * _shift(x, dx, dy) for w, (dx, dy) in zip(ws, shifts))
        Z = sum(ws)
        return (U / Z, Z) if return_D else (U / Z, None)

    def _KT_action(self, y, guide=None, sig=None):
        ws, shifts = self._weights(y, guide, sig)
        return sum(torch.roll(w * y, shifts=(dx, dy), dims=(-2, -1))
                   for w, (dx, dy) in zip(ws, shifts))

    def NLM_transpose(self, x, guide=None, sig=None, return_D=False):
        ws, _ = self._weights(x, guide, sig)
        D = sum(ws)
        out = self._KT_action(x / D.clamp_min(1e-6), guide=x if guide is None else guide,
                              sig=sig)
        return (out, D) if return_D else (out, None)

    def laplacian_grw(self, x, guide, sig=None, eps=1e-10):
        Wx, Z = self.forward(x, guide=guide, sig=sig)
        z = x - Wx
        return z - self._KT_action(z / Z.clamp_min(1e-6), guide=guide, sig=sig)


class FakeMetropolis(nn.Module, _HeadMixMixin):
    """Metropolis NeKDe: half-plane weights through the symmetric Metropolis
    construction (the package's direct statement, pinned by the CPU suite)."""

    def __init__(self, C=3, R=2, heads=2, comp_box=True, seed=0):
        super().__init__()
        self.window_rad = R
        self.comp_box = comp_box
        self.metropolis_eps = 1e-6
        self.features = _Features(C, 2 * heads, seed)
        self._setup_heads(C, heads, seed, "softmax")

    def _normalise_sigma(self, x, sig):
        return sig

    def pre_activation(self, x, sigma=None):
        return self.features(x, sigma)

    def _collect_shifts(self):
        return _halfplane(self.window_rad)

    def _halfplane_weights(self, phi, padded_phi, sig, shift_list):
        R = self.window_rad
        H, W = phi.shape[-2:]
        return [0.1 * torch.sigmoid(_head_scores(
            phi, padded_phi[:, :, R + dx:R + dx + H, R + dy:R + dy + W], self.n_heads))
            for dx, dy, _ in shift_list]

    def _head_mix_matrix(self):
        return _mix_matrix(self)

    def _mix_heads(self, w, C, mat):
        return self._mix(w, C)

    def forward(self, x, guide=None, sig=None, return_D=False):
        R = self.window_rad
        phi = self.pre_activation(x if guide is None else guide, sigma=sig)
        padded = F.pad(phi, (R, R, R, R), mode="circular")
        shifts = self._collect_shifts()
        C = x.shape[1]
        w_half = torch.stack([self._mix(w, C) for w in
                              self._halfplane_weights(phi, padded, sig, shifts)], dim=1)
        from neural_shift_cuda.metropolis import metropolis_aggregate_torch
        Wx, dh = metropolis_aggregate_torch(w_half, x, shifts, self.comp_box, 1e-6)
        return (Wx, dh) if return_D else (Wx, None)


class FakeNECTR(nn.Module):
    """Official NECTR contract: concat head over (guide, shifted guide)
    pairs, half-plane with box-masked mirrors, U / Z."""

    def __init__(self, C=2, R=2, latent=4, activation="control_sigmoid", seed=0):
        super().__init__()
        torch.manual_seed(seed)
        self.window_rad = R
        self.model_type = "concat"
        self.output_activation = activation
        self.sigma = 1.5
        self.lat = nn.Conv2d(C, latent, 1).double()
        self.proj = nn.ModuleList([nn.ModuleList([
            nn.Conv2d(2 * latent, latent, 1), nn.LayerNorm(latent), nn.LeakyReLU()])]).double()
        out_dim = 3 * C if activation == "control_sigmoid" else C
        self.out = nn.Conv2d(latent, out_dim, 1, bias=False).double()

    def pre_activation(self, x, sigma=None):
        return self.lat(x)

    def controlled_sigmoid(self, k, a, b):
        return F.softplus(a) / (1 + torch.exp(-torch.sigmoid(b) * k))

    def N_theta(self, g, g_s):
        v = torch.cat((g, g_s), dim=1)
        for block in self.proj:
            for i, layer in enumerate(block):
                v = layer(v.permute(0, 2, 3, 1)).permute(0, 3, 1, 2) if i == 1 else layer(v)
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
        for dx, dy, inv in _halfplane(self.window_rad):
            if cache is None:
                w = self.N_theta(g, _shift(g, dx, dy)) * _box(H, W, dx, dy, x)
                held[(dx, dy)] = w
            else:
                w = cache[(dx, dy)]
            U = U + w * _shift(x, dx, dy)
            Z = Z + w
            if inv:
                wi = torch.roll(w, shifts=(dx, dy), dims=(-2, -1)) * _box(H, W, -dx, -dy, x)
                U = U + wi * _shift(x, -dx, -dy)
                Z = Z + wi
        return (U / Z, Z, held) if store_cache else (U / Z, Z)


class FakeNekre(FakeNECTR):
    """Legacy batched contract."""

    def forward(self, x, guide=None, sig=None, batched=False):
        return FakeNECTR.forward(self, x, reference=guide, sig=sig)


def _fresh(cls, **kw):
    """A subclass per test so installs do not leak between tests."""
    sub = type(cls.__name__ + "Case", (cls,), {})
    return sub, sub(**kw)


def _inputs(B=2, C=3, H=9, W=10, dtype=torch.float64, seed=5, device="cpu"):
    g = torch.Generator().manual_seed(seed)
    x = torch.rand(B, C, H, W, generator=g, dtype=torch.float64)
    guide = torch.rand(B, C, H, W, generator=g, dtype=torch.float64)
    return x.to(dtype).to(device), guide.to(dtype).to(device)
