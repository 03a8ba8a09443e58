"""Comparison helpers and independent dense restatements used as pins.

The dense restatements build each operator as an explicit matrix on tiny
images (pixel loops in Python), so they share no code path with the oracle's
gather loops or the HIP kernels; torch autograd through them yields the
gradients.
"""
from __future__ import annotations

import torch


def assert_bound(actual: torch.Tensor, expected: torch.Tensor, scale: torch.Tensor,
                 rtol: float, what: str = "", out_ulp: float = 0.0) -> None:
    """Error-bound-aware comparison.

    |actual - expected| <= rtol * (|expected| + scale) + out_ulp * |expected|
    elementwise, where `scale` is the sum of absolute values of the terms
    that formed each element (so cancellation near zero does not make a
    correct sum fail a plain relative test) and `out_ulp` covers the final
    rounding of a low-precision output.  Results computed in fp32 also get
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
    tol = (rtol * (e.abs() + s) + out_ulp * e.abs() + floor)[fin]
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


def box_np(H: int, W: int, dx: int, dy: int) -> torch.Tensor:
    m = torch.zeros(H, W, dtype=torch.float64)
    for h in range(H):
        for w in range(W):
            m[h, w] = 1.0 if (_in(h + dx, H) and _in(w + dy, W)) else 0.0
    return m


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
