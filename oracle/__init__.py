"""CPU oracle for the shift-window operators -- TEST INFRASTRUCTURE ONLY.

This package wraps ``oracle/oracle.c`` (a plain-C restatement of the
reference algorithm, built by ``oracle/Makefile`` into ``oracle/_build``).
Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker; the product package
``neural_shift_cuda_amd`` never touches it.

Every function takes and returns contiguous CPU ``torch`` tensors (used here
purely as typed host buffers) and names the reference code it restates
(paths relative to the reference repository root):

==========================  =====================================================
function                    reference
==========================  =====================================================
shift_gather                neural_shift_cuda/ops.py:95-135 (shift_gather_reference)
pair_gather                 neural_shift_cuda/ops.py:138-154 (pair_gather_reference)
shift_gather_bwd            adjoint of the above; csrc/shift_ops_cuda.cu:165-203
pair_gather_bwd             adjoint of pair_gather_reference
accumulate_uz               neural_shift_cuda/ops.py:157-206 (term order + _tree_sum)
accumulate_uz_bwd           csrc/shift_ops_cuda.cu:343-458 (analytic adjoint)
normalized                  ops.py:234-320 (policy "cpu"); shift_ops_cuda.cu:474-653
                            (policy "gpu")
normalized_bwd              csrc/shift_ops_cuda.cu:505-525, 655-791
metropolis                  csrc/metropolis_cuda.cu:70-186, metropolis.py:54-114
accumulate_uz_scalar(_bwd)  ops.py:350-390, csrc/shift_ops_cuda.cu:806-980
==========================  =====================================================

Parity pins for each function live in ``tests/test_oracle.py``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional, Tuple

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib: Optional[ctypes.CDLL] = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_D = ctypes.c_double


def build() -> str:
    """Compile the oracle with its Makefile (idempotent)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        for name in ("nso_shift_gather_fwd", "nso_pair_gather_fwd"):
            getattr(lib, name).argtypes = [_P, _I64, _P, _I64, _I64, _I64, _I64,
                                           _I64, _I64, _P, _P, _P, _P]
            getattr(lib, name).restype = None
        for suf in ("f32", "f64"):
            for name in ("nso_shift_gather_bwd", "nso_pair_gather_bwd"):
                fn = getattr(lib, f"{name}_{suf}")
                fn.argtypes = [_P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P]
                fn.restype = None
            fn = getattr(lib, f"nso_accumulate_uz_fwd_{suf}")
            fn.argtypes = [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _P]
            fn.restype = _I
            fn = getattr(lib, f"nso_accumulate_uz_bwd_{suf}")
            fn.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
                           _P, _P]
            fn.restype = None
            fn = getattr(lib, f"nso_normalized_fwd_{suf}")
            fn.argtypes = [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I, _I,
                           _P, _P]
            fn.restype = _I
            fn = getattr(lib, f"nso_normalized_bwd_{suf}")
            fn.argtypes = [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                           _I64, _I, _P, _P]
            fn.restype = None
            fn = getattr(lib, f"nso_metropolis_fwd_{suf}")
            fn.argtypes = [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I, _D,
                           _P, _P, _P]
            fn.restype = _I
            fn = getattr(lib, f"nso_accumulate_uz_scalar_fwd_{suf}")
            fn.argtypes = [_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P]
            fn.restype = _I
            fn = getattr(lib, f"nso_accumulate_uz_scalar_bwd_{suf}")
            fn.argtypes = [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
                           _I64, _P, _P]
            fn.restype = None
        lib.nso_set_num_threads.argtypes = [_I]
        lib.nso_set_num_threads.restype = None
        lib.nso_max_threads.argtypes = []
        lib.nso_max_threads.restype = _I
        _lib = lib
    return _lib


def set_num_threads(n: int) -> None:
    _load().nso_set_num_threads(int(n))


def max_threads() -> int:
    return int(_load().nso_max_threads())


def _host(t: torch.Tensor, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    t = t.detach().cpu()
    if dtype is not None:
        t = t.to(dtype)
    return t.contiguous()


def _shifts(shifts, cols: Optional[int] = None) -> torch.Tensor:
    t = torch.as_tensor(shifts).detach().cpu().to(torch.int64).contiguous()
    if t.dim() != 2 or t.size(1) not in (2, 3):
        raise ValueError(f"shifts must be (S, 2) or (S, 3); got {tuple(t.shape)}")
    if cols is not None and t.size(1) != cols:
        raise ValueError(f"shifts must have {cols} columns")
    return t


def _suffix(dtype: torch.dtype) -> Tuple[str, torch.dtype]:
    if dtype == torch.float64:
        return "f64", torch.float64
    if dtype == torch.float32:
        return "f32", torch.float32
    raise TypeError(f"oracle arithmetic runs in float32 or float64, not {dtype}")


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# ---------------------------------------------------------------------------
# gathers (bit-exact byte copies, any dtype)
# ---------------------------------------------------------------------------

def _gather(name: str, guide: torch.Tensor, shifts, pair: bool):
    g = _host(guide)
    sh = _shifts(shifts)
    B, C, H, W = g.shape
    S = sh.size(0)
    out = torch.empty((S * B, 2 * C if pair else C, H, W), dtype=g.dtype)
    mask = torch.empty((S * B, 1, H, W), dtype=g.dtype)
    one = torch.ones(1, dtype=g.dtype)
    zero = torch.zeros(1, dtype=g.dtype)
    getattr(_load(), name)(g.data_ptr(), g.element_size(), sh.data_ptr(), S,
                           sh.size(1), B, C, H, W, out.data_ptr(),
                           mask.data_ptr(), one.data_ptr(), zero.data_ptr())
    return out, mask


def shift_gather(guide: torch.Tensor, shifts):
    """(gs, mask) with gs[s*B+b] = guide[b] gathered at (h+dx, w+dy) mod."""
    return _gather("nso_shift_gather_fwd", guide, shifts, False)


def pair_gather(guide: torch.Tensor, shifts):
    """(pair, mask); pair[s*B+b] = cat(guide[b], shifted guide[b])."""
    return _gather("nso_pair_gather_fwd", guide, shifts, True)


def _gather_bwd(name: str, gout: torch.Tensor, shifts, B, C, H, W, dtype):
    suf, dt = _suffix(dtype)
    go = _host(gout, dt)
    sh = _shifts(shifts)
    g = torch.empty((B, C, H, W), dtype=dt)
    getattr(_load(), f"{name}_{suf}")(go.data_ptr(), sh.data_ptr(), sh.size(0),
                                      sh.size(1), B, C, H, W, g.data_ptr())
    return g


def shift_gather_bwd(gout, shifts, B, C, H, W, dtype=torch.float64):
    return _gather_bwd("nso_shift_gather_bwd", gout, shifts, B, C, H, W, dtype)


def pair_gather_bwd(gout, shifts, B, C, H, W, dtype=torch.float64):
    return _gather_bwd("nso_pair_gather_bwd", gout, shifts, B, C, H, W, dtype)


# ---------------------------------------------------------------------------
# accumulate_uz
# ---------------------------------------------------------------------------

def accumulate_uz(x, w, shifts, dtype=torch.float64):
    """(U, Z) in the reference CPU fallback's term order and tree."""
    suf, dt = _suffix(dtype)
    xh, wh = _host(x, dt), _host(w, dt)
    sh = _shifts(shifts, 3)
    B, C, H, W = xh.shape
    S = sh.size(0)
    if wh.shape != (S * B, C, H, W):
        raise ValueError(f"weights must be {(S * B, C, H, W)}")
    U = torch.empty_like(xh)
    Z = torch.empty_like(xh)
    rc = getattr(_load(), f"nso_accumulate_uz_fwd_{suf}")(
        xh.data_ptr(), wh.data_ptr(), sh.data_ptr(), S, B, C, H, W,
        U.data_ptr(), Z.data_ptr())
    if rc != 0:
        raise MemoryError("oracle accumulate_uz: allocation failed")
    return U, Z


def accumulate_uz_bwd(x, w, gU, gZ, shifts, dtype=torch.float64):
    """(gx, gw): analytic adjoint of accumulate_uz."""
    suf, dt = _suffix(dtype)
    xh, wh, gu, gz = (_host(t, dt) for t in (x, w, gU, gZ))
    sh = _shifts(shifts, 3)
    B, C, H, W = xh.shape
    S = sh.size(0)
    gx = torch.empty_like(xh)
    gw = torch.empty_like(wh)
    getattr(_load(), f"nso_accumulate_uz_bwd_{suf}")(
        xh.data_ptr(), wh.data_ptr(), gu.data_ptr(), gz.data_ptr(),
        sh.data_ptr(), S, B, C, H, W, gx.data_ptr(), gw.data_ptr())
    return gx, gw


# ---------------------------------------------------------------------------
# normalized_accumulate_uz
# ---------------------------------------------------------------------------

_POLICY = {"cpu": 0, "gpu": 1}


def normalized(x, w, shifts, *, log_weights: bool, policy: str = "gpu",
               dtype=torch.float64):
    """(D, log_C).  policy "cpu" restates the reference CPU fallback,
    "gpu" the reference GPU kernel (they differ only for negative positive
    weights: masked vs NaN)."""
    suf, dt = _suffix(dtype)
    xh, wh = _host(x, dt), _host(w, dt)
    sh = _shifts(shifts, 3)
    B, C, H, W = xh.shape
    S = sh.size(0)
    D = torch.empty_like(xh)
    L = torch.empty_like(xh)
    rc = getattr(_load(), f"nso_normalized_fwd_{suf}")(
        xh.data_ptr(), wh.data_ptr(), sh.data_ptr(), S, B, C, H, W,
        int(bool(log_weights)), _POLICY[policy], D.data_ptr(), L.data_ptr())
    if rc != 0:
        raise MemoryError("oracle normalized: allocation failed")
    return D, L


def normalized_bwd(x, w, D, L, gD, gL, shifts, *, log_weights: bool,
                   dtype=torch.float64):
    suf, dt = _suffix(dtype)
    xh, wh, Dh, Lh, gd, gl = (_host(t, dt) for t in (x, w, D, L, gD, gL))
    sh = _shifts(shifts, 3)
    B, C, H, W = xh.shape
    S = sh.size(0)
    gx = torch.empty_like(xh)
    gw = torch.empty_like(wh)
    getattr(_load(), f"nso_normalized_bwd_{suf}")(
        xh.data_ptr(), wh.data_ptr(), Dh.data_ptr(), Lh.data_ptr(),
        gd.data_ptr(), gl.data_ptr(), sh.data_ptr(), S, B, C, H, W,
        int(bool(log_weights)), gx.data_ptr(), gw.data_ptr())
    return gx, gw


# ---------------------------------------------------------------------------
# Metropolis
# ---------------------------------------------------------------------------

def metropolis(w_half, img, shifts, use_box: bool, eps: float = 1e-6,
               dtype=torch.float64, return_degree: bool = False):
    """(Wx, d_hat[, d]) for batch-major w_half (B, S, C, H, W)."""
    suf, dt = _suffix(dtype)
    wh, xh = _host(w_half, dt), _host(img, dt)
    sh = _shifts(shifts, 3)
    B, S, C, H, W = wh.shape
    if sh.size(0) != S:
        raise ValueError("shift table length must equal w_half.size(1)")
    Wx = torch.empty_like(xh)
    dh = torch.empty_like(xh)
    d = torch.empty_like(xh)
    rc = getattr(_load(), f"nso_metropolis_fwd_{suf}")(
        wh.data_ptr(), xh.data_ptr(), sh.data_ptr(), B, S, C, H, W,
        int(bool(use_box)), float(eps), Wx.data_ptr(), dh.data_ptr(),
        d.data_ptr())
    if rc != 0:
        raise MemoryError("oracle metropolis: allocation failed")
    return (Wx, dh, d) if return_degree else (Wx, dh)


# ---------------------------------------------------------------------------
# accumulate_uz_scalar
# ---------------------------------------------------------------------------

def accumulate_uz_scalar(x, w, shifts, dtype=torch.float64):
    """(U, Z) for per-(s, b, c) scalar weights w of shape (S, B, C)."""
    suf, dt = _suffix(dtype)
    xh, wh = _host(x, dt), _host(w, dt)
    sh = _shifts(shifts)
    B, C, H, W = xh.shape
    S = sh.size(0)
    U = torch.empty_like(xh)
    Z = torch.empty_like(xh)
    rc = getattr(_load(), f"nso_accumulate_uz_scalar_fwd_{suf}")(
        xh.data_ptr(), wh.data_ptr(), sh.data_ptr(), sh.size(1), S, B, C, H, W,
        U.data_ptr(), Z.data_ptr())
    if rc != 0:
        raise MemoryError("oracle accumulate_uz_scalar: allocation failed")
    return U, Z


def accumulate_uz_scalar_bwd(x, w, gU, gZ, shifts, dtype=torch.float64):
    suf, dt = _suffix(dtype)
    xh, wh, gu, gz = (_host(t, dt) for t in (x, w, gU, gZ))
    sh = _shifts(shifts)
    B, C, H, W = xh.shape
    S = sh.size(0)
    gx = torch.empty_like(xh)
    gw = torch.empty_like(wh)
    getattr(_load(), f"nso_accumulate_uz_scalar_bwd_{suf}")(
        xh.data_ptr(), wh.data_ptr(), gu.data_ptr(), gz.data_ptr(),
        sh.data_ptr(), sh.size(1), S, B, C, H, W, gx.data_ptr(), gw.data_ptr())
    return gx, gw


# ---------------------------------------------------------------------------
# Window evaluation (crops of images too large for the full oracle)
# ---------------------------------------------------------------------------

def window_indices(n: int, start: int, halo: int, length: int) -> torch.Tensor:
    """Global indices (start - halo + i) mod n, i < length + 2*halo."""
    return (torch.arange(length + 2 * halo, dtype=torch.int64) + (start - halo)) % n


def take_window(t: torch.Tensor, gh0: int, gw0: int, ch: int, cw: int, halo: int) -> torch.Tensor:
    """The (..., ch+2*halo, cw+2*halo) wrapped window of the last two dims of
    `t` (any device) as a contiguous CPU tensor."""
    H, W = t.shape[-2], t.shape[-1]
    rows = window_indices(H, gh0, halo, ch).to(t.device)
    cols = window_indices(W, gw0, halo, cw).to(t.device)
    return t.index_select(-2, rows).index_select(-1, cols).cpu().contiguous()


def _wlib(name: str, suf: str):
    lib = _load()
    fn = getattr(lib, f"{name}_{suf}")
    return fn


def accumulate_uz_window(xw, ww, shifts, halo, H, W, gh0, gw0, ch, cw, dtype=torch.float64):
    suf, dt = _suffix(dtype)
    xh, wh = _host(xw, dt), _host(ww, dt)
    sh = _shifts(shifts, 3)
    B, C = xh.shape[0], xh.shape[1]
    S = sh.size(0)
    fn = _wlib("nso_accumulate_uz_window_fwd", suf)
    fn.argtypes = [_P, _P, _P] + [_I64] * 10 + [_P, _P]
    fn.restype = _I
    U = torch.empty(B, C, ch, cw, dtype=dt)
    Z = torch.empty_like(U)
    rc = fn(xh.data_ptr(), wh.data_ptr(), sh.data_ptr(), S, B, C, halo, H, W, gh0, gw0, ch, cw,
            U.data_ptr(), Z.data_ptr())
    if rc != 0:
        raise MemoryError("oracle window accumulate failed")
    return U, Z


def accumulate_uz_window_bwd(xw, ww, gUw, gZw, shifts, halo, H, W, gh0, gw0, ch, cw,
                             dtype=torch.float64):
    suf, dt = _suffix(dtype)
    xh, wh, gu, gz = (_host(t, dt) for t in (xw, ww, gUw, gZw))
    sh = _shifts(shifts, 3)
    B, C = xh.shape[0], xh.shape[1]
    S = sh.size(0)
    fn = _wlib("nso_accumulate_uz_window_bwd", suf)
    fn.argtypes = [_P] * 5 + [_I64] * 10 + [_P, _P]
    fn.restype = None
    gx = torch.empty(B, C, ch, cw, dtype=dt)
    gw = torch.empty(S * B, C, ch, cw, dtype=dt)
    fn(xh.data_ptr(), wh.data_ptr(), gu.data_ptr(), gz.data_ptr(), sh.data_ptr(), S, B, C, halo,
       H, W, gh0, gw0, ch, cw, gx.data_ptr(), gw.data_ptr())
    return gx, gw


def metropolis_window(whw, imgw, shifts, halo, H, W, gh0, gw0, ch, cw, use_box, eps=1e-6,
                      dtype=torch.float64):
    """Window Metropolis; the halo must be >= 2*max|shift|."""
    suf, dt = _suffix(dtype)
    wh, xh = _host(whw, dt), _host(imgw, dt)
    sh = _shifts(shifts, 3)
    B, S, C = wh.shape[0], wh.shape[1], wh.shape[2]
    fn = _wlib("nso_metropolis_window", suf)
    fn.argtypes = [_P, _P, _P] + [_I64] * 10 + [_I, _D, _P, _P]
    fn.restype = _I
    Wx = torch.empty(B, C, ch, cw, dtype=dt)
    dh = torch.empty_like(Wx)
    rc = fn(wh.data_ptr(), xh.data_ptr(), sh.data_ptr(), B, S, C, halo, H, W, gh0, gw0, ch, cw,
            int(bool(use_box)), float(eps), Wx.data_ptr(), dh.data_ptr())
    if rc != 0:
        raise ValueError("oracle metropolis window: halo must be >= 2*max|shift|")
    return Wx, dh
