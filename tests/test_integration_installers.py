"""Model installers (neural_shift_cuda.integration) against small stand-in
model classes whose own methods state the operator directly (per-shift
loops over torch.roll), in the manner of the reference's
tests/test_cached_forward_patches.py (SimpleNamespace caches).

On the CPU the patched GPU paths are called directly (the ops run their CPU
paths); the gpu-marked tests install the patches and call the patched
methods on cuda:0.  fp64 tolerances (1e-10) on the CPU; fp32 (2e-5) on the
GPU.
"""
from __future__ import annotations

import sys
from types import SimpleNamespace

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from neural_shift_cuda.integration import gasd_drunet_attn_patch as gasd_patch
from neural_shift_cuda.integration import nectr_patch
from neural_shift_cuda.integration import nekde_drunet_attn_patch as nekde_patch
from neural_shift_cuda.integration import nkd_metropolis_attn_patch as mp_patch
from neural_shift_cuda.metropolis import metropolis_aggregate_torch

HAS_GPU = torch.cuda.is_available()


def _case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


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


def _close(a, b, rtol=1e-10, atol=1e-12):
    torch.testing.assert_close(a.double().cpu(), b.double().cpu(), rtol=rtol, atol=atol)


# ---------------------------------------------------------------------------
# Cached fixed-guide paths (SimpleNamespace caches)
# ---------------------------------------------------------------------------

DEVICES = ["cpu", pytest.param("cuda", marks=[
    pytest.mark.gpu, pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")])]


def _cached_weights(x, shifts, use_box, scale=1.0, seed=1):
    g = torch.Generator().manual_seed(seed)
    H, W = x.shape[-2:]
    out = []
    for s in shifts:
        dx, dy = s[0], s[1]
        w = (torch.rand(x.shape, generator=g, dtype=torch.float64).to(x.dtype).to(x.device) + 0.1)
        w = w * scale
        if use_box:
            w = w * _box(H, W, dx, dy, x)
        out.append(w)
    return out


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("use_box", [True, False])
def test_nekde_forward_cached(device, use_box):
    if device == "cuda":
        _case(f"nekde cached cuda box={use_box}")
    x, _ = _inputs(device=device, dtype=torch.float32 if device == "cuda" else torch.float64)
    shifts = _halfplane(1)
    ws = _cached_weights(x, shifts, use_box)
    U, Z = _symmetric_serial(x, ws, shifts, use_box)
    cache = SimpleNamespace(C=x.shape[1], shifts=shifts, w_fwd_list=ws, comp_box=use_box, D=Z)
    model = SimpleNamespace()
    out, deg = nekde_patch._forward_cached_cuda(model, x, cache, True)
    tol = dict(rtol=2e-5, atol=2e-6) if device == "cuda" else {}
    _close(out, U / Z.clamp_min(1e-6), **tol)
    assert deg is Z
    packed = model._nekde_parallel_weight_cache[4]
    nekde_patch._forward_cached_cuda(model, x, cache, False)
    assert model._nekde_parallel_weight_cache[4] is packed
    # without a cached degree the normalized reduction supplies it
    cache.D = None
    _, deg2 = nekde_patch._forward_cached_cuda(SimpleNamespace(), x, cache, True)
    _close(deg2, Z, **tol)


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("use_box", [True, False])
def test_gasd_cached_forward_transpose_laplacian(device, use_box):
    if device == "cuda":
        _case(f"gasd cached cuda box={use_box}")
    x, y = _inputs(device=device, dtype=torch.float32 if device == "cuda" else torch.float64)
    shifts = [(dx, dy) for dx in range(-1, 2) for dy in range(-1, 2)]
    ws = _cached_weights(x, shifts, use_box, seed=2)
    Z = sum(ws)
    Kx = sum(w * _shift(x, dx, dy) for w, (dx, dy) in zip(ws, shifts))
    KTy = sum(torch.roll(w * y, shifts=(dx, dy), dims=(-2, -1)) for w, (dx, dy) in zip(ws, shifts))
    cache = SimpleNamespace(C=x.shape[1], shifts=shifts, w_list=ws, Z=Z)
    model = SimpleNamespace()
    out, deg = gasd_patch._forward_cached_cuda(model, x, cache, True)
    tol = dict(rtol=2e-5, atol=2e-6) if device == "cuda" else {}
    _close(out, Kx / Z, **tol)
    assert deg is Z
    _close(gasd_patch._kt_action_cached_cuda(model, y, cache), KTy, **tol)
    z = x - Kx / Z
    KTz = sum(torch.roll(w * (z / Z.clamp_min(1e-6)), shifts=(dx, dy), dims=(-2, -1))
              for w, (dx, dy) in zip(ws, shifts))
    _close(gasd_patch._laplacian_grw_cached_cuda(model, x, cache), z - KTz, **tol)
    # a new cache object repacks and drops the transpose pack
    t_pack = model._gasd_parallel_transpose_cache[4]
    cache2 = SimpleNamespace(**vars(cache))
    gasd_patch._forward_cached_cuda(model, x, cache2, False)
    assert model._gasd_parallel_transpose_cache is None
    gasd_patch._kt_action_cached_cuda(model, y, cache2)
    assert model._gasd_parallel_transpose_cache[4] is not t_pack


@pytest.mark.parametrize("device", DEVICES)
@pytest.mark.parametrize("use_box", [True, False])
def test_metropolis_forward_cached(device, use_box):
    if device == "cuda":
        _case(f"metropolis cached cuda box={use_box}")
    x, _ = _inputs(device=device, dtype=torch.float32 if device == "cuda" else torch.float64)
    shifts = _halfplane(1)
    ws = _cached_weights(x, shifts, use_box, scale=0.08, seed=3)
    khat_x, dh = _symmetric_serial(x, ws, shifts, use_box)
    cache = SimpleNamespace(C=x.shape[1], shifts=shifts, w_hat_fwd_list=ws, comp_box=use_box,
                            degree_hat=dh)
    out, deg = mp_patch._forward_cached_cuda(SimpleNamespace(), x, cache, True)
    tol = dict(rtol=2e-5, atol=2e-6) if device == "cuda" else {}
    _close(out, x - dh * x + khat_x, **tol)
    assert deg is dh


def test_cached_argument_errors():
    x, _ = _inputs()
    shifts = _halfplane(1)
    ws = _cached_weights(x, shifts, True)
    with pytest.raises(ValueError, match="channels"):
        nekde_patch._forward_cached_cuda(
            SimpleNamespace(), x, SimpleNamespace(C=5, shifts=shifts, w_fwd_list=ws,
                                                  comp_box=True), True)
    with pytest.raises(ValueError, match="one tensor per cached shift"):
        nekde_patch._forward_cached_cuda(
            SimpleNamespace(), x, SimpleNamespace(C=3, shifts=shifts, w_fwd_list=ws[:-1],
                                                  comp_box=True), True)
    with pytest.raises(ValueError, match="identical"):
        gasd_patch._forward_cached_cuda(
            SimpleNamespace(), x, SimpleNamespace(C=3, shifts=[(0, 1)], w_list=[ws[0][:1]],
                                                  Z=None), True)
    with pytest.raises(ValueError, match="device and dtype"):
        mp_patch._forward_cached_cuda(
            SimpleNamespace(), x, SimpleNamespace(C=3, shifts=[(0, 1, True)],
                                                  w_hat_fwd_list=[ws[0].float()],
                                                  comp_box=True, degree_hat=None), True)


# ---------------------------------------------------------------------------
# NeKDe / GASD / Metropolis patched paths against the classes' own methods
# ---------------------------------------------------------------------------

NEKDE_CASES = [
    dict(comp_box=True), dict(comp_box=False), dict(activation="control_sigmoid"),
    dict(legacy=True), dict(legacy=True, comp_box=False, activation="control_sigmoid"),
    dict(heads=1, pos_act="none"), dict(heads=3, pos_act="none"), dict(pos_act="softplus"),
    dict(pos_act="relu"),
]


@pytest.mark.parametrize("kw", NEKDE_CASES)
def test_nekde_forward_and_transpose(kw):
    _, m = _fresh(FakeNeKDe, **kw)
    if kw.get("pos_act") == "relu":
        # every channel keeps a positive mix entry (an all-zero row would make
        # the class's U / Z 0/0, where the normalized op returns 0)
        with torch.no_grad():
            m.raw_head_mix.abs_().add_(0.1)
    x, guide = _inputs()
    m.train()
    D, Z = nekde_patch._forward_cuda(m, x, guide=guide, sig=0.1)
    rD, rZ = m.forward(x, guide=guide, sig=torch.tensor(0.1, dtype=torch.float64))
    _close(D, rD)
    _close(Z, rZ)
    m.eval()
    D2, none = nekde_patch._forward_cuda(m, x, return_D=False)
    assert none is None and m.max_batch_shifts is None
    _close(D2, m.forward(x)[0])
    for apply in (False, True):
        U, Zk = nekde_patch._kt_action_cuda(m, x, guide=guide, return_D=True, apply_Dinv=apply)
        rU, rZk = m._KT_action(x, guide=guide, return_D=True, apply_Dinv=apply)
        _close(U, rU)
        _close(Zk, rZk)


@pytest.mark.parametrize("kw", [dict(comp_box=True), dict(comp_box=False), dict(legacy=True),
                                dict(activation="control_sigmoid", heads=1, pos_act="none")])
def test_gasd_forward_transpose_laplacian(kw):
    _, m = _fresh(FakeGASD, **kw)
    x, guide = _inputs(seed=6)
    D, Z = gasd_patch._forward_cuda(m, x, guide=guide)
    rD, rZ = m.forward(x, guide=guide)
    _close(D, rD)
    _close(Z, rZ)
    _close(gasd_patch._kt_action_cuda(m, x, guide=guide), m._KT_action(x, guide=guide))
    WT, Dt = gasd_patch._nlm_transpose_cuda(m, x, guide=guide, return_D=True)
    rWT, rDt = m.NLM_transpose(x, guide=guide, return_D=True)
    _close(WT, rWT)
    _close(Dt, rDt)
    _close(gasd_patch._laplacian_grw_cuda(m, x, guide), m.laplacian_grw(x, guide))


@pytest.mark.parametrize("comp_box", [True, False])
def test_metropolis_forward(comp_box):
    _, m = _fresh(FakeMetropolis, comp_box=comp_box)
    x, guide = _inputs(seed=7)
    Wx, dh = mp_patch._forward_cuda(m, x, guide=guide, return_D=True)
    rW, rdh = m.forward(x, guide=guide, return_D=True)
    _close(Wx, rW)
    _close(dh, rdh)
    with pytest.raises(ValueError, match="same shape"):
        mp_patch._forward_cuda(m, x, guide=guide[:1])


def test_installers_dispatch_and_idempotence():
    """CPU inputs and use_cuda_shift=False keep the class's methods; the
    return_D default comes from the wrapped signature; a second install is a
    no-op."""
    from neural_shift_cuda.integration import (install_cuda_shift_attn, install_cuda_shift_gasd,
                                               install_cuda_shift_metropolis)
    x, guide = _inputs()
    for cls, inst in ((FakeNeKDe, install_cuda_shift_attn), (FakeGASD, install_cuda_shift_gasd),
                      (FakeMetropolis, install_cuda_shift_metropolis)):
        sub, m = _fresh(cls)
        before = m.forward(x, guide=guide)
        assert inst(sub) is sub
        patched = sub.forward
        assert inst(sub) is sub and sub.forward is patched
        after = m.forward(x, guide=guide)       # CPU: the class's own forward
        _close(after[0], before[0])
        if cls is FakeMetropolis:
            assert after[1] is None             # return_D defaults to False there
        else:
            _close(after[1], before[1])
        m.use_cuda_shift = False
        _close(m.forward(x, guide=guide)[0], before[0])
    sub, m = _fresh(FakeGASD)
    install_cuda_shift_gasd(sub)
    _close(m.NLM_transpose(x)[0], FakeGASD.NLM_transpose(m, x)[0])


def test_installer_without_transpose_raises_on_cpu():
    """A class without its own _KT_action gets the patched one, which has
    nothing to fall back to for CPU inputs."""
    from neural_shift_cuda.integration import install_cuda_shift_attn
    Bare = type("Bare", (nn.Module,), {"forward": FakeNeKDe.forward})
    install_cuda_shift_attn(Bare)
    inst = Bare()
    with pytest.raises(AttributeError, match="no reference _KT_action"):
        inst._KT_action(torch.zeros(1, 1, 4, 4))


# ---------------------------------------------------------------------------
# NECTR
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("activation", ["control_sigmoid", "exp", "raw"])
@pytest.mark.parametrize("pair", [True, False])
def test_nectr_official_forward_and_cache(activation, pair):
    from neural_shift_cuda.integration import install_cuda_shift_nectr
    sub, m = _fresh(FakeNECTR, activation=activation)
    x, ref = _inputs(C=2, seed=8)
    rD, rZ, rcache = m.forward(x, reference=ref, store_cache=True)
    install_cuda_shift_nectr(sub)
    m.use_cuda_pair_gather = pair
    D, Z, cache = m.forward(x, reference=ref, store_cache=True)
    _close(D, rD, rtol=1e-9)
    _close(Z, rZ, rtol=1e-9)
    kind = {"control_sigmoid": "positive", "exp": "log", "raw": "raw"}[activation]
    assert isinstance(cache, nectr_patch.NECTRWeightCache) and cache.weight_kind == kind
    # the patched forward's own cache, and a cache of the class's forward
    D2, Z2 = m.forward(x, cache=cache)
    _close(D2, rD, rtol=1e-9)
    D3, Z3 = m.forward(x, cache=rcache)
    _close(D3, rD, rtol=1e-9)
    _close(Z3, rZ, rtol=1e-9)
    m.use_cuda_shift = False
    _close(m.forward(x, reference=ref)[0], rD)


def test_nectr_legacy_and_contract():
    from neural_shift_cuda.integration import install_cuda_shift_nectr
    sub, m = _fresh(FakeNekre)
    x, g = _inputs(C=2, seed=9)
    rD, rZ = m.forward(x, guide=g)
    install_cuda_shift_nectr(sub)
    assert install_cuda_shift_nectr(sub) is sub
    D, Z = m.forward(x, guide=g, batched=True)
    _close(D, rD, rtol=1e-9)
    _close(Z, rZ, rtol=1e-9)
    D2, _ = m.forward(x, guide=g)           # batched defaults to False: own forward
    _close(D2, rD)

    class Other(nn.Module):
        def forward(self, x, y):
            return x
    with pytest.raises(TypeError, match="forward contract"):
        install_cuda_shift_nectr(Other)


# ---------------------------------------------------------------------------
# GPU: installed patches on cuda:0
# ---------------------------------------------------------------------------

def _to(m, device, dtype):
    return m.to(device=device, dtype=dtype)


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
@pytest.mark.parametrize("kw", [dict(comp_box=True), dict(comp_box=False), dict(legacy=True),
                                dict(heads=1, pos_act="none"),
                                dict(heads=1, pos_act="none", comp_box=False)])
def test_gpu_nekde_installed(kw):
    from neural_shift_cuda.integration import install_cuda_shift_attn
    _case(f"installed nekde {kw}")
    sub, m = _fresh(FakeNeKDe, **kw)
    x, guide = _inputs(H=24, W=20)
    rD, rZ = m.forward(x, guide=guide)
    rU, _ = m._KT_action(x, guide=guide, apply_Dinv=True)
    install_cuda_shift_attn(sub)
    _to(m, "cuda", torch.float32)
    xc, gc = x.float().cuda(), guide.float().cuda()
    D, Z = m.forward(xc, guide=gc)
    _close(D, rD, rtol=2e-5, atol=2e-6)
    _close(Z, rZ, rtol=2e-5, atol=2e-6)
    U, _ = m._KT_action(xc, guide=gc, apply_Dinv=True)
    _close(U, rU, rtol=2e-5, atol=2e-6)


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
@pytest.mark.parametrize("comp_box,heads", [(True, 2), (False, 2), (True, 1)])
def test_gpu_gasd_installed(comp_box, heads):
    from neural_shift_cuda.integration import install_cuda_shift_gasd
    _case(f"installed gasd box={comp_box} heads={heads}")
    sub, m = _fresh(FakeGASD, comp_box=comp_box, heads=heads)
    x, guide = _inputs(H=24, W=20, seed=10)
    rD, rZ = m.forward(x, guide=guide)
    rKT = m._KT_action(x, guide=guide)
    rL = m.laplacian_grw(x, guide)
    install_cuda_shift_gasd(sub)
    _to(m, "cuda", torch.float32)
    xc, gc = x.float().cuda(), guide.float().cuda()
    D, Z = m.forward(xc, guide=gc)
    _close(D, rD, rtol=2e-5, atol=2e-6)
    _close(m._KT_action(xc, guide=gc), rKT, rtol=2e-5, atol=2e-6)
    _close(m.laplacian_grw(xc, gc), rL, rtol=2e-5, atol=2e-5)


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
@pytest.mark.parametrize("comp_box", [True, False])
def test_gpu_metropolis_installed_with_grad(comp_box):
    """Installed Metropolis forward on the GPU, and its gradients (the shape
    is below the fused backward's minimum, so the explicit-edge path runs)."""
    from neural_shift_cuda.integration import install_cuda_shift_metropolis
    _case(f"installed metropolis box={comp_box}")
    sub, m = _fresh(FakeMetropolis, comp_box=comp_box)
    x, guide = _inputs(H=24, W=20, seed=11)
    xr = x.clone().requires_grad_(True)
    rW, _ = m.forward(xr, guide=guide)
    rW.sum().backward()
    install_cuda_shift_metropolis(sub)
    _to(m, "cuda", torch.float32)
    xc = x.float().cuda().requires_grad_(True)
    Wx, none = m.forward(xc, guide=guide.float().cuda())
    assert none is None
    _close(Wx, rW, rtol=2e-5, atol=2e-6)
    Wx.sum().backward()
    _close(xc.grad, xr.grad, rtol=1e-4, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
@pytest.mark.parametrize("activation", ["control_sigmoid", "exp"])
def test_gpu_nectr_installed(activation):
    from neural_shift_cuda.integration import install_cuda_shift_nectr
    _case(f"installed nectr {activation}")
    sub, m = _fresh(FakeNECTR, activation=activation)
    x, ref = _inputs(C=2, H=24, W=20, seed=12)
    rD, rZ = m.forward(x, reference=ref)
    install_cuda_shift_nectr(sub)
    _to(m, "cuda", torch.float32)
    D, Z = m.forward(x.float().cuda(), reference=ref.float().cuda())
    _close(D, rD, rtol=2e-5, atol=2e-6)
    _close(Z, rZ, rtol=2e-5, atol=2e-6)


# ---------------------------------------------------------------------------
# NECTR installer on the vendored official model: golden vectors written by
# tests/golden/make_golden.py from models/NECTR_models1.py and the
# reference's own installer (integration/nectr_patch.py)
# ---------------------------------------------------------------------------

def _nectr_golden_names():
    from helpers import golden_names
    return golden_names("nectr_installer")


def _nectr_golden(name, device="cpu"):
    from helpers import golden_cases
    from nectr_fixture import NECTRGoldenModel, from_golden
    case = golden_cases()[name]
    sub = type("NECTRGoldenCase", (NECTRGoldenModel,), {})
    model, x, sig = from_golden(case)
    model.__class__ = sub
    model = model.to(device)
    return case, sub, model, x.to(device), (None if sig is None else sig.to(device))


@pytest.mark.parametrize("name", _nectr_golden_names())
def test_nectr_golden_official_model(name):
    """The stand-in model equals the official model's own forward, and the
    installed forward equals the reference installer's output on it (from
    the guide and from the unpatched forward's cache)."""
    from neural_shift_cuda.integration import install_cuda_shift_nectr
    case, sub, model, x, sig = _nectr_golden(name)
    O = case["outputs"]
    with torch.no_grad():
        D0, Z0, cache0 = model(x, sig=sig, store_cache=True)
        _close(D0, O["D_model"], rtol=1e-12, atol=1e-14)
        _close(Z0, O["Z_model"], rtol=1e-12, atol=1e-14)
        install_cuda_shift_nectr(sub)
        D1, Z1, cache1 = model(x, sig=sig, store_cache=True)
        assert cache1.weight_kind == case["cache_weight_kind"]
        _close(D1, O["D_patched"], rtol=1e-12, atol=1e-14)
        _close(Z1, O["Z_patched"], rtol=1e-12, atol=1e-14)
        D2, Z2 = model(x, sig=sig, cache=cache0)
        _close(D2, O["D_plain_cache"], rtol=1e-12, atol=1e-14)
        _close(Z2, O["Z_plain_cache"], rtol=1e-12, atol=1e-14)
        D3, Z3 = model(x, sig=sig, cache=cache1)
        _close(D3, O["D_patched"], rtol=1e-12, atol=1e-14)
    if not model.blind:
        with pytest.raises(ValueError, match="sigma is None"):
            model(x, cache=cache0)


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
@pytest.mark.parametrize("name", _nectr_golden_names())
def test_gpu_nectr_golden_official_model(name):
    """The installed forward on cuda:0 (fp64 HIP kernels) against the
    reference installer's output on the official model."""
    from neural_shift_cuda.integration import install_cuda_shift_nectr
    _case(f"nectr golden {name}")
    case, sub, model, x, sig = _nectr_golden(name, "cuda")
    install_cuda_shift_nectr(sub)
    O = case["outputs"]
    with torch.no_grad():
        D, Z = model(x, sig=sig)
        _close(D, O["D_patched"], rtol=1e-10, atol=1e-12)
        _close(Z, O["Z_patched"], rtol=1e-10, atol=1e-12)
        model.use_cuda_pair_gather = False
        D, Z = model(x, sig=sig)
        _close(D, O["D_patched"], rtol=1e-10, atol=1e-12)


def test_channel_operand_detects_broadcast():
    """Single-head stacks reach the ops as one shared plane per (shift,
    batch); mixed stacks stay per channel."""
    from neural_shift_cuda_amd.integration._common import channel_operand, mix_heads
    w = torch.rand(5, 2, 1, 6, 7)
    op, shared = channel_operand(mix_heads(w, 3, None))
    assert shared and op.shape == (10, 1, 6, 7) and torch.equal(op, w.reshape(10, 1, 6, 7))
    op, shared = channel_operand(mix_heads(torch.rand(5, 2, 3, 6, 7), 3, None))
    assert not shared and op.shape == (10, 3, 6, 7)


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a GPU")
@pytest.mark.parametrize("comp_box", [True, False])
def test_gpu_nekde_single_head_gradients(comp_box):
    """Training through the installed single-head NeKDe forward: the shared
    weight planes' gradient (the channel sum of the kernels' per-channel
    gradient) reaches the model's parameters as through the class's own
    forward."""
    from neural_shift_cuda.integration import install_cuda_shift_attn
    _case(f"nekde single head gradients box={comp_box}")
    sub, m = _fresh(FakeNeKDe, heads=1, pos_act="none", comp_box=comp_box)
    x, guide = _inputs(H=24, W=20, seed=13)
    m.train()
    rD, _ = m.forward(x, guide=guide)
    rD.pow(2).sum().backward()
    ref = {n: p.grad.clone() for n, p in m.named_parameters() if p.grad is not None}
    assert ref
    m.zero_grad()
    install_cuda_shift_attn(sub)
    _to(m, "cuda", torch.float32)
    D, _ = m.forward(x.float().cuda(), guide=guide.float().cuda())
    _close(D, rD, rtol=2e-5, atol=2e-6)
    D.pow(2).sum().backward()
    for n, p in m.named_parameters():
        if n in ref:
            _close(p.grad, ref[n], rtol=2e-4, atol=2e-5)
