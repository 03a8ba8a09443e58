"""Comparison helpers and independent dense restatements used as pins.

The dense restatements build each operator as an explicit matrix on tiny
images (pixel loops in Python), so they share no code path with the oracle's
gather loops or the HIP kernels; torch autograd through them yields the
gradients.
"""
from __future__ import annotations

import torch


def assert_bound(actual: torch.Tensor, expected: torch.Tensor, scale: torch.Tensor,
                 rtol: float, what: str = "", out_ulp: float = 0.0,
                 extra: torch.Tensor = None) -> None:
    """Error-bound-aware comparison.

    |actual - expected| <= rtol * (|expected| + scale) + out_ulp * |expected|
                           + extra
    elementwise, where `scale` is the sum of absolute values of the terms
    that formed each element (so cancellation near zero does not make a
    correct sum fail a plain relative test), `out_ulp` covers the final
    rounding of a low-precision output and `extra` (optional, absolute) is
    an error term propagated from a factor whose own error is not O(rtol)
    (see normalized_bwd_cond).  Results computed in fp32 also get
    an absolute floor of 2^-110 for terms below fp32's normal range (an
    exp(-160) term is 0 in fp32 but 1e-70 in the fp64 oracle), and fp16
    outputs one fp16 subnormal step.  NaN
    positions must coincide and infinities must match exactly.
    """
    floor = 2.0 ** -110 if actual.dtype != torch.float64 else 0.0
    if actual.dtype == torch.float16:
        floor = 2.0 ** -24  # fp16 subnormal spacing: outputs below it round to 0
    a = actual.detach().to(torch.float64).cpu()
    e = expected.detach().to(torch.float64).cpu()
    s = scale.detach().to(torch.float64).cpu().abs()
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} vs {tuple(e.shape)}"
    an, en = torch.isnan(a), torch.isnan(e)
    assert torch.equal(an, en), f"{what}: NaN pattern differs ({int((an ^ en).sum())} elements)"
    ai, ei = torch.isinf(a), torch.isinf(e)
    assert torch.equal(ai, ei) and torch.equal(a[ai], e[ei]), f"{what}: infinities differ"
    fin = ~(an | ai)
    err = (a - e).abs()[fin]
    tol = rtol * (e.abs() + s) + out_ulp * e.abs() + floor
    if extra is not None:
        x = extra.detach().to(torch.float64).cpu().abs()
        assert x.shape == e.shape, f"{what}: extra shape {tuple(x.shape)}"
        assert bool(torch.isfinite(x[fin]).all()), f"{what}: non-finite extra bound"
        tol = tol + x
    tol = tol[fin]
    if err.numel():
        worst = (err / tol.clamp_min(1e-300)).max().item()
        idx = int((err / tol.clamp_min(1e-300)).argmax())
        assert worst <= 1.0, (
            f"{what}: max err/tol = {worst:.3g} (err {err[idx].item():.3g}, "
            f"tol {tol[idx].item():.3g}, rtol {rtol})")


def rtol_for(dtype: torch.dtype) -> float:
    """Accumulation tolerance: 1e-5 relative for fp32-accumulated inputs,
    1e-12 for fp64 (of the per-element term scale)."""
    return 1e-12 if dtype == torch.float64 else 1e-5


def out_ulp_for(dtype: torch.dtype) -> float:
    """Half an ulp of a low-precision output plus margin."""
    return {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}.get(dtype, 0.0)


def _scratch_device():
    """Where the fp64 bound evaluations run: the GPU when there is one (they
    are plain torch ops, independent of the kernels under test)."""
    return torch.device("cuda:0") if torch.cuda.is_available() else torch.device("cpu")


def unit_roundoff(dtype: torch.dtype) -> float:
    """u of the accumulator type: 2^-53 for fp64 inputs, 2^-24 otherwise."""
    return 2.0 ** -53 if dtype == torch.float64 else 2.0 ** -24


def _row_terms(w: torch.Tensor, shifts, s: int):
    """(forward key, mirror key, mirror box) of shift row s for every output
    pixel o: the forward term of o has key w_s[o]; the mirror term of an
    inverse row has key w_s[o - s] and exists where o - s is inside the
    image (the oracle's table semantics: any nonzero has_inverse)."""
    dx, dy, inv = (int(v) for v in shifts[s].tolist())
    H, W = w.shape[-2:]
    if not inv:
        return w[s], None, None
    box = box_np(H, W, -dx, -dy, w.device).to(w.dtype)
    return w[s], roll_gather(w[s], -dx, -dy), box


def normalized_bwd_cond(x, w, L, gD, gL, Ds, shifts, *, log_weights: bool,
                        acc_dtype: torch.dtype):
    """Per-element error term of the normalized backward that comes from the
    conditioning of its fractions f = exp(l - L) (log weights) and
    F = exp(-L) (positive weights), as the `extra` of assert_bound.

    Every gradient term is a fraction times a factor: gx sums f * gD[o],
    gw sums F * score(o, v).  The kernels evaluate the fraction from their
    own forward's L, so a fraction's relative error is
        kappa = dL_o + (error of evaluating exp at l - L_o)
    where, with u the unit roundoff of the accumulator type, n_o the number
    of valid terms of output pixel o and range_o = max l - min l over them:
      * log weights: the forward's online softmax forms each a_i and each
        rescale factor as exp(-|k - m|) (argument rounding |k - m| u / 2,
        then x log2(e) and exp2, about 1.5 |k - m| u + u); the rescales
        telescope to at most range_o; the positive fma sums add n_o u; the
        log and the final m + log z add 2 log(n_o) u + |L_o| u / 2.  So
        dL_o <= u (3 range_o + n_o + |L_o| + 2 log n_o + 4), and the
        backward's exp(l - L) adds u (|l - L_o| / 2 + 1).
      * positive weights: the scaling is by exact powers of two (scatter
        path) or one divide per term (gather path), so
        dL_o <= u (2 n_o + 3 |L_o| + 4 log n_o + 8), and w exp(-L) adds 2u.
    The extra bound is sum over terms of kappa * |fraction| * |factor|, with
    |score| <= |gD| (|v| + Ds) + |gLogC| (Ds >= |D| as in the scale).  The
    summation error of the backward itself stays under rtol * scale.
    x, w, L, gD, gL, Ds are the oracle-side tensors (L the fp64 oracle's
    log_C); shifts as the oracle takes them.  Returns (gx_extra, gw_extra)
    on the CPU."""
    u = unit_roundoff(acc_dtype)
    d64 = torch.float64
    dev = _scratch_device()
    B, C, H, W = x.shape
    S = int(shifts.size(0))
    shifts = shifts.cpu()
    x = x.to(dev, d64).abs()
    gD = gD.to(dev, d64).abs()
    gL = gL.to(dev, d64).abs()
    Ds = Ds.to(dev, d64).abs()
    L = L.to(dev, d64)
    w = w.to(dev, d64).reshape(S, B, C, H, W)
    ninf = float("-inf")

    def valid(k):
        if log_weights:
            return torch.isfinite(k)
        return (k > 0) & torch.isfinite(k)

    # pass 1: n_o and the logit range of every output pixel
    n = torch.zeros(B, C, H, W, dtype=d64, device=dev)
    kmax = torch.full((B, C, H, W), ninf, dtype=d64, device=dev)
    kmin = torch.full((B, C, H, W), float("inf"), dtype=d64, device=dev)
    for s in range(S):
        kf, km, box = _row_terms(w, shifts, s)
        for k, m in ((kf, None), (km, box)):
            if k is None:
                continue
            ok = valid(k) if m is None else valid(k) & (m > 0)
            n += ok.to(d64)
            if log_weights:
                kmax = torch.where(ok, torch.maximum(kmax, k), kmax)
                kmin = torch.where(ok, torch.minimum(kmin, k), kmin)
    fin_L = torch.isfinite(L)
    Lf = torch.where(fin_L, L, torch.zeros_like(L))
    logn = torch.log(n.clamp_min(1.0))
    if log_weights:
        rng = torch.where(n > 0, kmax - kmin, torch.zeros_like(n))
        dL = u * (3 * rng + n + Lf.abs() + 2 * logn + 4)
    else:
        dL = u * (2 * n + 3 * Lf.abs() + 4 * logn + 8)

    def frac_kappa(k, Lo, dLo, weight_grad):
        """|fraction| * kappa of a term with key k at an output with log C Lo."""
        ok = valid(k) & torch.isfinite(Lo)
        ks = torch.where(ok, k, torch.zeros_like(k))
        Ls = torch.where(ok, Lo, torch.zeros_like(Lo))
        if log_weights:
            f = torch.exp(ks - Ls)
            kap = dLo + u * (0.5 * (ks - Ls).abs() + 1)
        else:
            f = torch.exp(-Ls) if weight_grad else ks * torch.exp(-Ls)
            kap = dLo + 2 * u
        return torch.where(ok, f * kap, torch.zeros_like(f))

    gx = torch.zeros(B, C, H, W, dtype=d64, device=dev)
    gw = torch.zeros(S, B, C, H, W, dtype=d64, device=dev)
    for s in range(S):
        dx, dy, inv = (int(v) for v in shifts[s].tolist())
        v = w[s]
        # forward term of output q (reads x[q+s]): gx[q+s] += f gD[q]
        gx += torch.roll(frac_kappa(v, L, dL, False) * gD, (dx, dy), (-2, -1))
        g = frac_kappa(v, L, dL, True) * (gD * (roll_gather(x, dx, dy) + Ds) + gL)
        if inv:
            # mirror term of output q+s (inside the image) reads x[q]
            bx = box_np(H, W, dx, dy, dev)
            Ls, dLs = roll_gather(L, dx, dy), roll_gather(dL, dx, dy)
            gDs, gLs, Dss = roll_gather(gD, dx, dy), roll_gather(gL, dx, dy), roll_gather(Ds, dx, dy)
            gx += bx * frac_kappa(v, Ls, dLs, False) * gDs
            g = g + bx * frac_kappa(v, Ls, dLs, True) * (gDs * (x + Dss) + gLs)
        gw[s] = torch.where(valid(v), g, torch.zeros_like(g))
    return gx.cpu(), gw.reshape(S * B, C, H, W).cpu()


def metropolis_grad_abs(w_half, img, gWx, gdh, shifts, use_box: bool, eps: float = 1e-6):
    """Absolute-value evaluation of the Metropolis gradients, per element.

    The loss is <gWx, Wx> + <gdh, d_hat> with Wx = x - d_hat x + K_hat x.
    With a = gWx, b = gdh - gWx x, for the edge of pixel p towards j
    (forward j = p + s with weight wf_s[p] = w_s[p] box(+s); mirror
    j = p - s with weight wf_s[p - s] box(-s)), m = max(d_p, d_j, eps),
    wk = omega / m and G = a_p x_j + b_p:
        d loss / d omega  = G / m
        d loss / d m      = -G wk / m      (to d_p, d_j by the max rule,
                                            0 below eps)
        d loss / d x_j   += wk a_p,   d loss / d x_p += a_p (1 - d_hat_p)
    and d = sum of every edge weight at its pixel, so
        grad w_s[q] = box_f[q] (G_f[q] / m + gd[q])
                    + [inv] box_f[q] box_i[q+s] (G_i[q+s] / m + gd[q+s]).
    This evaluates the same expressions with |a|, |b| <= |gdh| + |a||x|,
    |x| and the absolute value of every contribution, in fp64: the sum of
    |terms| behind each gradient element, the scale of assert_bound.
    Returns (w_half scale (B, S, C, H, W), img scale (B, C, H, W)) on the
    CPU."""
    d64 = torch.float64
    dev = _scratch_device()
    B, S, C, H, W = w_half.shape
    w = w_half.to(dev, d64)
    x = img.to(dev, d64)
    a = gWx.to(dev, d64).abs()
    ax = x.abs()
    babs = gdh.to(dev, d64).abs() + a * ax

    def box(dx, dy):
        return box_np(H, W, dx, dy, dev) if use_box else torch.ones(H, W, dtype=d64, device=dev)

    rows = [(int(dx), int(dy), bool(inv)) for dx, dy, inv in shifts]
    fwd, mir = [], []
    d = torch.zeros(B, C, H, W, dtype=d64, device=dev)
    for s, (dx, dy, inv) in enumerate(rows):
        wf = w[:, s] * box(dx, dy)
        fwd.append(wf)
        d = d + wf
        if inv:
            wi = torch.roll(wf, (dx, dy), (-2, -1)) * box(-dx, -dy)
            mir.append(wi)
            d = d + wi
        else:
            mir.append(None)

    def edge(omega, ex, ey):
        """(|d loss/d omega|, |d loss/d m| to p, to j, wk) for the edge p -> p + (ex, ey)."""
        dj = roll_gather(d, ex, ey)
        mx = torch.maximum(d, dj)
        m = mx.clamp_min(eps)
        wk = omega / m
        G = a * roll_gather(ax, ex, ey) + babs
        gm = G * wk / m * (mx >= eps).to(d64)
        sel = torch.where(d > dj, torch.ones_like(d),
                          torch.where(d == dj, torch.full_like(d, 0.5), torch.zeros_like(d)))
        return G / m, gm * sel, gm * (1 - sel), wk

    gd = torch.zeros_like(d)
    dh = torch.zeros_like(d)
    gxe = torch.zeros_like(d)  # sum of wk a_p over the edges that read x_j
    gom_f, gom_i = [], []
    for s, (dx, dy, inv) in enumerate(rows):
        go, gp, gj, wk = edge(fwd[s], dx, dy)
        gom_f.append(go)
        gd += gp + torch.roll(gj, (dx, dy), (-2, -1))
        dh += wk
        gxe += torch.roll(wk * a, (dx, dy), (-2, -1))
        if inv:
            go, gp, gj, wk = edge(mir[s], -dx, -dy)
            gom_i.append(go)
            gd += gp + torch.roll(gj, (-dx, -dy), (-2, -1))
            dh += wk
            gxe += torch.roll(wk * a, (-dx, -dy), (-2, -1))
        else:
            gom_i.append(None)
    gx = a * (1 + dh) + gxe
    gw = torch.zeros(B, S, C, H, W, dtype=d64, device=dev)
    for s, (dx, dy, inv) in enumerate(rows):
        g = box(dx, dy) * (gom_f[s] + gd)
        if inv:
            g = g + box(dx, dy) * roll_gather(box(-dx, -dy) * (gom_i[s] + gd), dx, dy)
        gw[:, s] = g
    return gw.cpu(), gx.cpu()


def metropolis_torch_ordered(w_half, img, shifts, use_box: bool, order, eps: float = 1e-6):
    """(Wx, d_hat) of the Metropolis operator, differentiable, with every
    edge's max(d_p, d_j) routed by a given degree ordering.

    The operator is the direct statement of reference metropolis.py:54-114
    (degree pass, then w / max(d_p, d_j, eps) per edge).  Only the max is
    changed: it is evaluated as sel d_p + (1 - sel) d_j with sel = 1, 1/2, 0
    as order_p >, ==, < order_j.  With `order` the degree in the inputs'
    own precision this is the function whose gradient a kernel that
    compares its own degrees computes: its value differs from the exact max
    only where the two orderings disagree, i.e. by less than the degree's
    rounding (|d_p - d_j| there), and torch.maximum's even split on exact
    ties is kept.  d_p, d_j themselves are the exact (input-dtype) degrees.
    """
    B, S, C, H, W = w_half.shape
    dt, dev = img.dtype, img.device
    order = order.to(dev, torch.float64)
    rows = [(int(dx), int(dy), bool(inv)) for dx, dy, inv in shifts]

    def box(dx, dy):
        return box_np(H, W, dx, dy, dev).to(dt) if use_box else None

    fwd, mir = [], []
    d = torch.zeros_like(img)
    for s, (dx, dy, inv) in enumerate(rows):
        k = box(dx, dy)
        wf = w_half[:, s] if k is None else w_half[:, s] * k
        fwd.append(wf)
        d = d + wf
        if inv:
            ki = box(-dx, -dy)
            wi = roll_gather(wf, -dx, -dy)
            wi = wi if ki is None else wi * ki
            mir.append(wi)
            d = d + wi
        else:
            mir.append(None)

    def edge_max(ex, ey):
        oj = roll_gather(order, ex, ey)
        sel = torch.where(order > oj, 1.0, torch.where(order == oj, 0.5, 0.0)).to(dt)
        return sel * d + (1 - sel) * roll_gather(d, ex, ey)

    kx = torch.zeros_like(img)
    dh = torch.zeros_like(img)
    for s, (dx, dy, inv) in enumerate(rows):
        wk = fwd[s] / edge_max(dx, dy).clamp_min(eps)
        kx = kx + wk * roll_gather(img, dx, dy)
        dh = dh + wk
        if inv:
            wk = mir[s] / edge_max(-dx, -dy).clamp_min(eps)
            kx = kx + wk * roll_gather(img, -dx, -dy)
            dh = dh + wk
    return img - dh * img + kx, dh


# ---------------------------------------------------------------------------
# Dense restatements (tiny images only)
# ---------------------------------------------------------------------------

def _in(v: int, n: int) -> bool:
    return 0 <= v < n


def accumulate_index(shifts, H: int, W: int):
    """Sparse pattern of the accumulate_uz operator of one (b, c) plane.

    Returns a list of (row p, column j, shift s, weight pixel q): the matrix
    K with K[p, j] += w_s[q] maps x to U (and 1 to Z).  Forward edges:
    p = q, j = (q+s) mod.  Mirror edges of has_inv rows: p = q + s
    (no wrap, inside the image), j = q.
    """
    ent = []
    for s, (dx, dy, inv) in enumerate(shifts):
        for h in range(H):
            for w in range(W):
                q = h * W + w
                ent.append((q, ((h + dx) % H) * W + (w + dy) % W, s, q))
                if inv and _in(h + dx, H) and _in(w + dy, W):
                    ent.append(((h + dx) * W + (w + dy), q, s, q))
    return ent


def dense_accumulate(x: torch.Tensor, w: torch.Tensor, shifts):
    """(U, Z) by explicit matrices; differentiable in x and w (fp64)."""
    B, C, H, W = x.shape
    S = len(shifts)
    N = H * W
    ent = accumulate_index(shifts, H, W)
    rows = torch.tensor([e[0] for e in ent])
    cols = torch.tensor([e[1] for e in ent])
    ss = torch.tensor([e[2] for e in ent])
    qq = torch.tensor([e[3] for e in ent])
    wv = w.reshape(S, B, C, N)
    U = torch.zeros(B, C, N, dtype=x.dtype)
    Z = torch.zeros(B, C, N, dtype=x.dtype)
    out_u, out_z = [], []
    for b in range(B):
        for c in range(C):
            K = torch.zeros(N, N, dtype=x.dtype).index_put(
                (rows, cols), wv[ss, b, c, qq], accumulate=True)
            xv = x[b, c].reshape(N)
            out_u.append(K @ xv)
            out_z.append(K.sum(1))
    U = torch.stack(out_u).reshape(B, C, H, W)
    Z = torch.stack(out_z).reshape(B, C, H, W)
    return U, Z


def dense_normalized(x: torch.Tensor, w: torch.Tensor, shifts, log_weights: bool):
    """(D, log_C) via per-pixel term lists and torch.logsumexp / softmax
    (positive weights enter as log w, masks as -inf); differentiable."""
    B, C, H, W = x.shape
    S = len(shifts)
    N = H * W
    ent = accumulate_index(shifts, H, W)
    per_row = [[] for _ in range(N)]
    for (p, j, s, q) in ent:
        per_row[p].append((j, s, q))
    T = max(len(r) for r in per_row)
    jj = torch.zeros(N, T, dtype=torch.long)
    ss = torch.zeros(N, T, dtype=torch.long)
    qq = torch.zeros(N, T, dtype=torch.long)
    valid = torch.zeros(N, T, dtype=torch.bool)
    for p, r in enumerate(per_row):
        for t, (j, s, q) in enumerate(r):
            jj[p, t], ss[p, t], qq[p, t], valid[p, t] = j, s, q, True
    wv = w.reshape(S, B, C, N)
    Ds, Ls = [], []
    for b in range(B):
        for c in range(C):
            k = wv[ss, b, c, qq]
            if log_weights:
                key = k
            else:
                pos = k > 0
                key = torch.where(pos, torch.where(pos, k, torch.ones_like(k)).log(),
                                  torch.full_like(k, float("-inf")))
            key = torch.where(valid, key, torch.full_like(key, float("-inf")))
            v = x[b, c].reshape(N)[jj]
            lse = torch.logsumexp(key, dim=1)
            empty = torch.isinf(lse) & (lse < 0)
            a = torch.softmax(torch.where(empty[:, None], torch.zeros_like(key), key), dim=1)
            a = torch.where(valid & ~empty[:, None], a, torch.zeros_like(a))
            Ds.append(torch.where(empty, torch.zeros_like(lse), (a * v).sum(1)))
            Ls.append(lse)
    return (torch.stack(Ds).reshape(B, C, H, W), torch.stack(Ls).reshape(B, C, H, W))


def dense_metropolis(w_half: torch.Tensor, img: torch.Tensor, shifts, use_box: bool,
                     eps: float):
    """(Wx, d_hat, W matrices) from explicit K, K_hat and W = I - diag(K_hat 1) + K_hat."""
    B, S, C, H, W = w_half.shape
    N = H * W
    Wxs, dhs, mats = [], [], []
    for b in range(B):
        for c in range(C):
            K = torch.zeros(N, N, dtype=img.dtype)
            for s, (dx, dy, inv) in enumerate(shifts):
                ws = w_half[b, s, c]
                for h in range(H):
                    for w in range(W):
                        p = h * W + w
                        if not use_box or (_in(h + dx, H) and _in(w + dy, W)):
                            K[p, ((h + dx) % H) * W + (w + dy) % W] += ws[h, w]
                        if inv and (not use_box or (_in(h - dx, H) and _in(w - dy, W))):
                            jh, jw = (h - dx) % H, (w - dy) % W
                            K[p, jh * W + jw] += ws[jh, jw]
            d = K.sum(1)
            den = torch.maximum(d[:, None], d[None, :]).clamp_min(eps)
            Kh = torch.where(K != 0, K / den, torch.zeros_like(K))
            dh = Kh.sum(1)
            Wm = torch.eye(N, dtype=img.dtype) - torch.diag(dh) + Kh
            Wxs.append(Wm @ img[b, c].reshape(N))
            dhs.append(dh)
            mats.append(Wm)
    return (torch.stack(Wxs).reshape(B, C, H, W), torch.stack(dhs).reshape(B, C, H, W), mats)


def roll_gather(t: torch.Tensor, dx: int, dy: int) -> torch.Tensor:
    """out[..., h, w] = t[..., (h+dx) mod H, (w+dy) mod W] via torch.roll."""
    return torch.roll(t, shifts=(-dx, -dy), dims=(-2, -1))


def box_np(H: int, W: int, dx: int, dy: int, device="cpu") -> torch.Tensor:
    """(H, W) fp64 indicator of 0 <= h + dx < H and 0 <= w + dy < W."""
    hs = torch.arange(H, device=device) + dx
    ws = torch.arange(W, device=device) + dy
    rows = (hs >= 0) & (hs < H)
    cols = (ws >= 0) & (ws < W)
    return (rows[:, None] & cols[None, :]).to(torch.float64)


# ---------------------------------------------------------------------------
# Golden vectors written by tests/golden/make_golden.py from the reference's
# own CPU fallbacks
# ---------------------------------------------------------------------------

_GOLDEN = None


def golden_cases():
    """{name: case} with case["inputs"] / case["outputs"] as CPU tensors."""
    global _GOLDEN
    if _GOLDEN is None:
        import json
        import os

        import numpy as np
        here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
        manifest = json.load(open(os.path.join(here, "golden.json")))
        arrays = np.load(os.path.join(here, "golden.npz"), allow_pickle=False)
        out = {}
        for case in manifest["cases"]:
            c = dict(case)
            for role in ("inputs", "outputs"):
                tens = {}
                for name, dt in case.get(role, {}).items():
                    a = torch.from_numpy(arrays[f"{case['name']}/{role}/{name}"].copy())
                    if dt == "bfloat16":
                        a = a.view(torch.bfloat16)
                    assert str(a.dtype).replace("torch.", "") == dt, (case["name"], name)
                    tens[name] = a
                c[role] = tens
            out[case["name"]] = c
        _GOLDEN = out
    return _GOLDEN


def golden_names(op: str):
    return sorted(n for n, c in golden_cases().items() if c["op"] == op)
